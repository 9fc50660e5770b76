"""Architecture cards of the two networks on the hot path, and the benchmark configurations.

DA3 variants follow depthanything3-rs/src/variant.rs:59-113 (dims, heads, depth, alt_start,
out_layers, head features and stage dims). MapAnything follows the compile-time constants of
mapanything-rs/src/{dinov2.rs:8-17, info_sharing.rs:12-14, dpt.rs:10-14, heads.rs:9-15}
("reference" spec) and the ViT-L / 768-wide info-sharing spec the benchmark configurations
name ("baseline_l" spec). The C structures in include/splathip.h carry the same fields.
"""
from __future__ import annotations

from dataclasses import dataclass, field, asdict
from typing import List, Tuple

PATCH = 14            # depthanything3-rs/src/variant.rs:9, mapanything-rs/src/dinov2.rs:7
HEAD_DIM = 64         # depthanything3-rs/src/variant.rs:11
TRAINED_GRID = 37     # depthanything3-rs/src/backbone.rs:21

IMAGENET_MEAN = (0.485, 0.456, 0.406)   # mapanything-rs/src/image_input.rs:113
IMAGENET_STD = (0.229, 0.224, 0.225)    # mapanything-rs/src/image_input.rs:114

FFN_MLP = 0      # fc2(gelu(fc1(x))), depthanything3-rs/src/vit_block.rs:70-79
FFN_SWIGLU = 1   # w3(silu(x1) * x2), mapanything-rs/src/vit_block.rs:48-71


def swiglu_hidden_dim(dim: int) -> int:
    """mapanything-rs/src/vit_block.rs:42-44: 2/3 of 4*dim rounded up to a multiple of 8."""
    return -(-(dim * 4 * 2 // 3) // 8) * 8


@dataclass(frozen=True)
class Da3Spec:
    name: str
    dim: int
    heads: int
    depth: int
    ffn: int
    alt_start: int
    out_layers: Tuple[int, int, int, int]
    head_features: int
    head_stage_dims: Tuple[int, int, int, int]

    @property
    def mlp_hidden(self) -> int:
        return swiglu_hidden_dim(self.dim) if self.ffn == FFN_SWIGLU else 4 * self.dim

    @property
    def head_input_dim(self) -> int:
        return 2 * self.dim


# depthanything3-rs/src/variant.rs:59-113; the index is the C ABI's `variant` argument.
DA3_VARIANTS = {
    "small": Da3Spec("small", 384, 6, 12, FFN_MLP, 4, (5, 7, 9, 11), 64, (48, 96, 192, 384)),
    "base": Da3Spec("base", 768, 12, 12, FFN_MLP, 4, (5, 7, 9, 11), 128, (96, 192, 384, 768)),
    "large": Da3Spec("large", 1024, 16, 24, FFN_MLP, 8, (11, 15, 19, 23), 256, (256, 512, 1024, 1024)),
    "giant": Da3Spec("giant", 1536, 24, 40, FFN_SWIGLU, 13, (19, 27, 33, 39), 256, (256, 512, 1024, 1024)),
}
DA3_VARIANT_INDEX = {"small": 0, "base": 1, "large": 2, "giant": 3}

# depthanything3-rs/src/reference_view.rs:21-29
REF_FIRST, REF_MIDDLE, REF_SADDLE = 0, 1, 2


@dataclass(frozen=True)
class MaSpec:
    """MapAnything widths. `enc_*` is the DINOv2 encoder, `info_*` the alternating-attention
    transformer; `hooks` are the info blocks whose normed output feeds the dense head (the
    last must be info_depth - 1). When enc_dim != info_dim a Linear(enc_dim -> info_dim)
    (`info_sharing.proj_embed`) maps the fused patch and class tokens into the info width."""
    name: str
    enc_dim: int
    enc_heads: int
    enc_depth: int
    enc_ffn: int
    enc_hidden: int
    info_dim: int
    info_heads: int
    info_depth: int
    info_ffn: int
    info_hidden: int
    hooks: Tuple[int, int, int]
    dpt_dims: Tuple[int, int, int, int] = (96, 192, 384, 768)
    dpt_features: int = 256
    pose_dim: int = 4 * PATCH * PATCH
    scale_dim: int = PATCH * PATCH

    @property
    def has_proj(self) -> bool:
        return self.enc_dim != self.info_dim


MA_SPECS = {
    # mapanything-rs/src/dinov2.rs:8-10 (ViT-giant truncated to 24 blocks, SwiGLU 4096),
    # info_sharing.rs:12-14 (16 blocks at 1536, hooks after 7 and 11 and the last).
    "reference": MaSpec("reference", 1536, 24, 24, FFN_SWIGLU, swiglu_hidden_dim(1536),
                        1536, 24, 16, FFN_SWIGLU, swiglu_hidden_dim(1536), (7, 11, 15)),
    # The benchmark's ViT-L/14 encoder and 24-block, 768-wide info transformer. Assumed: GELU
    # MLP ratio 4 in both, the 1024->768 projection, hooks after blocks 11, 17 and 23.
    "baseline_l": MaSpec("baseline_l", 1024, 16, 24, FFN_MLP, 4096,
                         768, 12, 24, FFN_MLP, 3072, (11, 17, 23)),
    # A small spec with the same topology, for parity tests the CPU oracle runs in seconds.
    "tiny": MaSpec("tiny", 128, 2, 3, FFN_MLP, 512, 128, 2, 4, FFN_MLP, 512, (1, 2, 3),
                   dpt_dims=(32, 64, 96, 128), dpt_features=64, pose_dim=96, scale_dim=48),
    "tiny_proj": MaSpec("tiny_proj", 192, 3, 3, FFN_MLP, 768, 128, 2, 4, FFN_SWIGLU,
                        swiglu_hidden_dim(128), (1, 2, 3),
                        dpt_dims=(32, 64, 96, 128), dpt_features=64, pose_dim=96, scale_dim=48),
    # The tiny transformer with the reference's 256-feature DPT head (its 128-channel output
    # convolution is the one whose epilogue runs the output head in bf16).
    "tiny_f256": MaSpec("tiny_f256", 128, 2, 3, FFN_MLP, 512, 128, 2, 4, FFN_MLP, 512, (1, 2, 3),
                        dpt_dims=(32, 64, 96, 128), dpt_features=256, pose_dim=96, scale_dim=48),
}


@dataclass(frozen=True)
class BenchConfig:
    key: str
    model: str            # "da3" or "ma"
    spec: str
    views: int
    height: int
    width: int
    dtype: str            # "f32", "bf16" or "f16"
    images: str           # "uniform" or "procedural"
    brightness: bool = False
    encoder_only: bool = False
    description: str = ""


# BASELINE.json "configs", in order.
CONFIGS = {
    "C1": BenchConfig("C1", "da3", "small", 1, 504, 504, "f32", "uniform",
                      description="DA3-Small, 1 view 504x504, fp32"),
    "C2": BenchConfig("C2", "da3", "small", 6, 378, 504, "bf16", "procedural",
                      description="DA3-Small, 6 views 378x504 (27x36 patches), bf16"),
    "C3": BenchConfig("C3", "ma", "baseline_l", 2, 392, 518, "bf16", "uniform", encoder_only=True,
                      description="MapAnything ViT-L/14 encoder only, 2 views 518x392, bf16"),
    "C4": BenchConfig("C4", "ma", "baseline_l", 6, 392, 518, "bf16", "procedural",
                      description="MapAnything (ViT-L enc, 24x768 info), 6 views 518x392, bf16"),
    "C5": BenchConfig("C5", "ma", "baseline_l", 24, 392, 518, "bf16", "procedural", brightness=True,
                      description="MapAnything (ViT-L enc, 24x768 info), 24 views 518x392, bf16"),
}
