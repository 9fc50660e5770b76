"""Seeded synthetic checkpoints and images for the benchmark configurations and the tests.

Checkpoints are written as safetensors under the reference's own key names, so the loader
reads them exactly as it would read a real checkpoint:
  * DA3: `model.` prefix, depthanything3-rs/src/weights.rs:16, keys from backbone.rs:69-91,
    vit_block.rs:127-145, dpt.rs:191-242, camera_head.rs:65-78;
  * MapAnything: no prefix, keys from mapanything-rs/src/{model.rs:69-81, dinov2.rs:90-101,
    vit_block.rs:83-95, info_sharing.rs:39-47, dpt.rs:147-182,254-273, heads.rs:55-121}.

Initialisation: matmul/conv weights and biases, pos/cls/camera/scale tokens and the view
embedding ~ N(0, 0.02); LayerNorm weight = 1 + N(0, 0.02), bias ~ N(0, 0.02); LayerScale
gammas = `layer_scale` (1e-5 for the benchmark configurations). Every tensor draws from its
own numpy PCG64 stream seeded by (seed, crc32(name)), so a tensor's values depend only on
the seed and its name.
"""
from __future__ import annotations

import math
import zlib
from typing import Dict, Tuple

import numpy as np

from .specs import (Da3Spec, MaSpec, FFN_SWIGLU, PATCH, TRAINED_GRID, HEAD_DIM,
                    IMAGENET_MEAN, IMAGENET_STD)

NORMAL, LN_WEIGHT, LN_BIAS, LAYER_SCALE = 0, 1, 2, 3
Shapes = Dict[str, Tuple[Tuple[int, ...], int]]


def _linear(out: Shapes, name: str, n_out: int, n_in: int, bias: bool = True) -> None:
    out[name + ".weight"] = ((n_out, n_in), NORMAL)
    if bias:
        out[name + ".bias"] = ((n_out,), NORMAL)


def _conv(out: Shapes, name: str, c_out: int, c_in: int, k: int, bias: bool = True) -> None:
    out[name + ".weight"] = ((c_out, c_in, k, k), NORMAL)
    if bias:
        out[name + ".bias"] = ((c_out,), NORMAL)


def _convt(out: Shapes, name: str, c_in: int, c_out: int, k: int) -> None:
    # ConvTranspose2d weight layout [in, out, kh, kw]
    out[name + ".weight"] = ((c_in, c_out, k, k), NORMAL)
    out[name + ".bias"] = ((c_out,), NORMAL)


def _ln(out: Shapes, name: str, n: int) -> None:
    out[name + ".weight"] = ((n,), LN_WEIGHT)
    out[name + ".bias"] = ((n,), LN_BIAS)


def _vit_block(out: Shapes, p: str, dim: int, ffn: int, hidden: int, qk_norm: bool) -> None:
    _ln(out, p + ".norm1", dim)
    _linear(out, p + ".attn.qkv", 3 * dim, dim)
    if qk_norm:
        _ln(out, p + ".attn.q_norm", HEAD_DIM)
        _ln(out, p + ".attn.k_norm", HEAD_DIM)
    _linear(out, p + ".attn.proj", dim, dim)
    out[p + ".ls1.gamma"] = ((dim,), LAYER_SCALE)
    _ln(out, p + ".norm2", dim)
    if ffn == FFN_SWIGLU:
        _linear(out, p + ".mlp.w12", 2 * hidden, dim)
        _linear(out, p + ".mlp.w3", dim, hidden)
    else:
        _linear(out, p + ".mlp.fc1", hidden, dim)
        _linear(out, p + ".mlp.fc2", dim, hidden)
    out[p + ".ls2.gamma"] = ((dim,), LAYER_SCALE)


def da3_shapes(spec: Da3Spec) -> Shapes:
    out: Shapes = {}
    d = spec.dim
    b = "model.backbone.pretrained"
    _conv(out, b + ".patch_embed.proj", d, 3, PATCH)
    out[b + ".cls_token"] = ((1, 1, d), NORMAL)
    out[b + ".camera_token"] = ((1, 2, d), NORMAL)
    out[b + ".pos_embed"] = ((1, 1 + TRAINED_GRID * TRAINED_GRID, d), NORMAL)
    _ln(out, b + ".norm", d)
    for i in range(spec.depth):
        _vit_block(out, f"{b}.blocks.{i}", d, spec.ffn, spec.mlp_hidden, i >= spec.alt_start)
    h = "model.head"
    hin, f = spec.head_input_dim, spec.head_features
    _ln(out, h + ".norm", hin)
    for k, c in enumerate(spec.head_stage_dims):
        _conv(out, f"{h}.projects.{k}", c, hin, 1)
        _conv(out, f"{h}.scratch.layer{k + 1}_rn", f, c, 3, bias=False)
    c0, c1, _, c3 = spec.head_stage_dims
    _convt(out, h + ".resize_layers.0", c0, c0, 4)
    _convt(out, h + ".resize_layers.1", c1, c1, 2)
    _conv(out, h + ".resize_layers.3", c3, c3, 3)
    for suffix in ("", "_aux"):
        for level in range(1, 5):
            p = f"{h}.scratch.refinenet{level}{suffix}"
            units = ("resConfUnit1", "resConfUnit2") if level < 4 else ("resConfUnit2",)
            for u in units:
                _conv(out, f"{p}.{u}.conv1", f, f, 3)
                _conv(out, f"{p}.{u}.conv2", f, f, 3)
            _conv(out, p + ".out_conv", f, f, 1)
    s = h + ".scratch"
    _conv(out, s + ".output_conv1", f // 2, f, 3)
    _conv(out, s + ".output_conv2.0", 32, f // 2, 3)
    _conv(out, s + ".output_conv2.2", 2, 32, 1)
    for i in range(5):
        cin, cout = (f, f // 2) if i % 2 == 0 else (f // 2, f)
        _conv(out, f"{s}.output_conv1_aux.3.{i}", cout, cin, 3)
    _conv(out, s + ".output_conv2_aux.3.0", 32, f // 2, 3)
    _conv(out, s + ".output_conv2_aux.3.5", 7, 32, 1)
    c = "model.cam_dec"
    _linear(out, c + ".backbone.0", hin, hin)
    _linear(out, c + ".backbone.2", hin, hin)
    _linear(out, c + ".fc_t", 3, hin)
    _linear(out, c + ".fc_qvec", 4, hin)
    _linear(out, c + ".fc_fov.0", 2, hin)
    return out


def ma_shapes(spec: MaSpec) -> Shapes:
    out: Shapes = {}
    e, d = spec.enc_dim, spec.info_dim
    p = "encoder.model"
    _conv(out, p + ".patch_embed.proj", e, 3, PATCH)
    out[p + ".cls_token"] = ((1, 1, e), NORMAL)
    out[p + ".pos_embed"] = ((1, 1 + TRAINED_GRID * TRAINED_GRID, e), NORMAL)
    for i in range(spec.enc_depth):
        _vit_block(out, f"{p}.blocks.{i}", e, spec.enc_ffn, spec.enc_hidden, False)
    _ln(out, "fusion_norm_layer", e)
    out["scale_token"] = ((d,), NORMAL)
    q = "info_sharing"
    if spec.has_proj:
        _linear(out, q + ".proj_embed", d, e)
    for i in range(spec.info_depth):
        _vit_block(out, f"{q}.self_attention_blocks.{i}", d, spec.info_ffn, spec.info_hidden, False)
    _ln(out, q + ".norm", d)
    out[q + ".view_pos_table"] = ((1, d), NORMAL)
    f = spec.dpt_features
    for h, c in enumerate(spec.dpt_dims):
        hp = f"dense_head.0.input_process.{h}"
        _conv(out, hp + ".0.0", c, e if h == 0 else d, 1)
        if h == 0:
            _convt(out, hp + ".0.1", c, c, 4)
        elif h == 1:
            _convt(out, hp + ".0.1", c, c, 2)
        elif h == 3:
            _conv(out, hp + ".0.1", c, c, 3)
        _conv(out, hp + ".1", f, c, 3, bias=False)
    for level in range(1, 5):
        rp = f"dense_head.0.scratch.refinenet{level}"
        units = ("resConfUnit1", "resConfUnit2") if level < 4 else ("resConfUnit2",)
        for u in units:
            _conv(out, f"{rp}.{u}.conv1", f, f, 3)
            _conv(out, f"{rp}.{u}.conv2", f, f, 3)
        _conv(out, rp + ".out_conv", f, f, 1)
    _conv(out, "dense_head.1.conv1", f // 2, f, 3)
    _conv(out, "dense_head.1.conv2.0", f // 2, f // 2, 3)
    _conv(out, "dense_head.1.conv2.2", 6, f // 2, 1)
    pd = spec.pose_dim
    _conv(out, "pose_head.proj", pd, d, 1)
    for blk in range(2):
        for k in range(1, 4):
            _conv(out, f"pose_head.res_conv.{blk}.res_conv{k}", pd, pd, 1)
    _linear(out, "pose_head.more_mlps.0", pd, pd)
    _linear(out, "pose_head.more_mlps.2", pd, pd)
    _linear(out, "pose_head.fc_t", 3, pd)
    _linear(out, "pose_head.fc_rot", 4, pd)
    sd = spec.scale_dim
    _linear(out, "scale_head.proj", sd, d)
    _linear(out, "scale_head.mlp.0.0", sd, sd)
    _linear(out, "scale_head.mlp.1.0", sd, sd)
    _linear(out, "scale_head.output_proj", 1, sd)
    # known-intrinsics ray encoder, mapanything-rs/src/ray_encoder.rs:56-76 (fixed widths)
    w0, w1, w2 = 3 * PATCH * PATCH, 768, 1024
    _conv(out, "ray_dirs_encoder.conv_in", w0, w0, 3)
    for i, (ci, co) in enumerate(((w0, w1), (w1, w2))):
        _conv(out, f"ray_dirs_encoder.encoder.{i}.conv1", co, ci, 3)
        _conv(out, f"ray_dirs_encoder.encoder.{i}.conv2", co, co, 3)
        _conv(out, f"ray_dirs_encoder.encoder.{i}.shortcut", co, ci, 1)
    _conv(out, "ray_dirs_encoder.encoder.2", e, w2, 1)
    _ln(out, "ray_dirs_encoder.norm_layer", e)
    return out


def _one(name: str, shape, kind: int, seed: int, layer_scale: float, std: float) -> np.ndarray:
    n = int(np.prod(shape))
    if kind == LAYER_SCALE:
        arr = np.full(n, layer_scale, dtype=np.float32)
    else:
        rng = np.random.default_rng([seed, zlib.crc32(name.encode())])
        arr = rng.standard_normal(n, dtype=np.float32)
        arr *= np.float32(std)
        if kind == LN_WEIGHT:
            arr += np.float32(1.0)
    return arr.reshape(shape)


def generate(shapes: Shapes, seed: int, layer_scale: float = 1e-5, std: float = 0.02,
             threads: int = 8) -> Dict[str, np.ndarray]:
    """Every tensor of `shapes`, in a thread pool (the values do not depend on the pool)."""
    from concurrent.futures import ThreadPoolExecutor
    names = list(shapes)
    with ThreadPoolExecutor(max_workers=max(1, threads)) as pool:
        arrays = list(pool.map(lambda k: _one(k, shapes[k][0], shapes[k][1], seed, layer_scale, std), names))
    return dict(zip(names, arrays))


def save(path: str, tensors: Dict[str, np.ndarray]) -> None:
    from safetensors.numpy import save_file
    save_file({k: np.ascontiguousarray(v) for k, v in tensors.items()}, path)


def load(path: str) -> Dict[str, np.ndarray]:
    from safetensors.numpy import load_file
    return load_file(path)


# ---------------------------------------------------------------------------------------
# Images: [V, 3, H, W] float32, ImageNet-normalised (mapanything-rs/src/image_input.rs:195-216)

def normalise(rgb01: np.ndarray) -> np.ndarray:
    mean = np.asarray(IMAGENET_MEAN, np.float32).reshape(1, 3, 1, 1)
    std = np.asarray(IMAGENET_STD, np.float32).reshape(1, 3, 1, 1)
    return ((rgb01.astype(np.float32) - mean) / std).astype(np.float32)


def uniform_images(views: int, height: int, width: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng([seed, 0x1A6E])
    return normalise(rng.random((views, 3, height, width), dtype=np.float32))


def procedural_images(views: int, height: int, width: int, seed: int,
                      brightness: bool = False, noise_sigma: float = 0.05) -> np.ndarray:
    """Smooth colour fields: per view and channel 0.5 + a sum of 4 seeded low-frequency
    sinusoids (amplitude 0.12 each, 0.5-3 periods across the image), plus uniform noise of
    standard deviation `noise_sigma`, clipped to [0, 1]; with `brightness` each view is also
    scaled by U[0.7, 1.3] before clipping."""
    rng = np.random.default_rng([seed, 0x9C0C])
    y = (np.arange(height, dtype=np.float64) + 0.5) / height
    x = (np.arange(width, dtype=np.float64) + 0.5) / width
    yy, xx = np.meshgrid(y, x, indexing="ij")
    out = np.empty((views, 3, height, width), np.float32)
    half_width = noise_sigma * math.sqrt(3.0)
    for v in range(views):
        for c in range(3):
            field = np.full((height, width), 0.5)
            for _ in range(4):
                fx, fy = rng.uniform(0.5, 3.0, 2) * rng.choice([-1.0, 1.0], 2)
                phase = rng.uniform(0, 2 * math.pi)
                field += 0.12 * np.sin(2 * math.pi * (fx * xx + fy * yy) + phase)
            out[v, c] = field
        out[v] += rng.uniform(-half_width, half_width, (3, height, width))
        if brightness:
            out[v] *= rng.uniform(0.7, 1.3)
    return normalise(np.clip(out, 0.0, 1.0))


def config_images(cfg, seed: int) -> np.ndarray:
    if cfg.images == "uniform":
        return uniform_images(cfg.views, cfg.height, cfg.width, seed)
    return procedural_images(cfg.views, cfg.height, cfg.width, seed, brightness=cfg.brightness)
