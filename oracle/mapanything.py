"""CPU oracle for MapAnything — TEST INFRASTRUCTURE ONLY (see oracle/common.py).

Restates mapanything-rs/src/{model,dinov2,vit_block,info_sharing,dpt,heads,ray_encoder}.rs
in torch-CPU float32, parameterised by a spec (splathip.specs.MaSpec) so that the reference's
constants and the benchmark's ViT-L / 768 widths both run. With enc_dim != info_dim the
assumed `info_sharing.proj_embed` Linear maps the fused patches and raw class token to
info_dim.
"""
from __future__ import annotations

from typing import Dict

import numpy as np
import torch
import torch.nn.functional as F

from . import common as C

LN_EPS = 1e-6           # mapanything-rs/src/vit_block.rs:8
RAY_MIN_NORM = 1e-8     # mapanything-rs/src/model.rs:17
CONF_MIN = 1.0          # mapanything-rs/src/model.rs:19
QUAT_MIN_NORM = 1e-8    # mapanything-rs/src/heads.rs:16
MIN_SCALE = 1e-8        # mapanything-rs/src/heads.rs:17
RAY_WIDTHS = (3 * 14 * 14, 768, 1024)  # mapanything-rs/src/ray_encoder.rs:11-12


def encoder_forward(p, spec, images, taps=None, branch_taps=None):
    """mapanything-rs/src/dinov2.rs:129-145, all views batched (each view is independent).
    branch_taps: per block, the [attention, feed-forward] branch outputs before LayerScale."""
    V, _, H, W = images.shape
    R, Cc = H // C.PATCH, W // C.PATCH
    e = "encoder.model"
    patches = C.conv(images, p, e + ".patch_embed.proj", stride=C.PATCH).flatten(2).transpose(1, 2)
    pos = C.positional_embedding(p[e + ".pos_embed"], R, Cc).to(images.dtype)
    xs = torch.cat([p[e + ".cls_token"].expand(V, 1, spec.enc_dim), patches], 1) + pos
    for i in range(spec.enc_depth):
        bt = [] if branch_taps is not None else None
        xs = C.vit_block(xs, p, f"{e}.blocks.{i}", spec.enc_ffn == 1, LN_EPS, taps=bt)
        if taps is not None:
            taps.append(xs.clone())
        if branch_taps is not None:
            branch_taps.append([t[1].clone() for t in bt])
    return xs


def info_sharing_forward(p, spec, patches, classes, taps=None, branch_taps=None):
    """mapanything-rs/src/info_sharing.rs:50-102. patches [V, P, d], classes [V, 1, d].
    branch_taps: per block, the [attention, feed-forward] branch outputs before LayerScale
    (a per-view block's cover the V*n view tokens only; the scale token waits)."""
    V, P, d = patches.shape
    n = P + 1
    q = "info_sharing"
    seq = torch.cat([patches, classes], 1)                       # per view [patches, class]
    seq = torch.cat([seq[:1] + p[q + ".view_pos_table"][0], seq[1:]], 0)
    xs = torch.cat([seq.reshape(1, V * n, d), p["scale_token"].reshape(1, 1, d)], 1)
    stored = []
    for i in range(spec.info_depth):
        name = f"{q}.self_attention_blocks.{i}"
        bt = [] if branch_taps is not None else None
        if i % 2 == 0:
            xs = C.vit_block(xs, p, name, spec.info_ffn == 1, LN_EPS, taps=bt)
        else:
            per_view = xs[:, :V * n].reshape(V, n, d)
            att = C.vit_block(per_view, p, name, spec.info_ffn == 1, LN_EPS, taps=bt).reshape(1, V * n, d)
            xs = torch.cat([att, xs[:, V * n:]], 1)
        if taps is not None:
            taps.append(xs.clone())
        if branch_taps is not None:
            branch_taps.append([t[1].clone() for t in bt])
        if i in spec.hooks:
            stored.append(C.layer_norm(xs, p[q + ".norm.weight"], p[q + ".norm.bias"], LN_EPS))
    per_view = [[s[0, v * n: v * n + P] for s in stored] for v in range(V)]
    return per_view, stored[2][0, V * n]


def _rcu(x, p, name):
    """mapanything-rs/src/dpt.rs:94-113"""
    out = C.conv(F.relu(x), p, name + ".conv1", padding=1)
    out = C.conv(F.relu(out), p, name + ".conv2", padding=1)
    return out + x


def _fusion(x, skip, p, name):
    """mapanything-rs/src/dpt.rs:116-140: out_conv(up2x(RCU2(x + RCU1(skip))))"""
    if skip is not None:
        x = x + _rcu(skip, p, name + ".resConfUnit1")
    y = _rcu(x, p, name + ".resConfUnit2")
    y = C.resize_bilinear(y, 2 * y.shape[2], 2 * y.shape[3])
    return C.conv(y, p, name + ".out_conv")


def dpt_forward(p, spec, hooks, R, Cc):
    """mapanything-rs/src/dpt.rs:174-199, views batched. hooks: 4 tensors [V, P, dim]."""
    pyr = []
    for h, tok in enumerate(hooks):
        V, P, D = tok.shape
        x = tok.transpose(1, 2).reshape(V, D, R, Cc)
        hp = f"dense_head.0.input_process.{h}"
        x = C.conv(x, p, hp + ".0.0")
        if h == 0:
            x = C.conv_t(x, p, hp + ".0.1", 4)
        elif h == 1:
            x = C.conv_t(x, p, hp + ".0.1", 2)
        elif h == 3:
            x = C.conv(x, p, hp + ".0.1", padding=1, stride=2)
        pyr.append(C.conv(x, p, hp + ".1", padding=1))
    path = _fusion(pyr[3], None, p, "dense_head.0.scratch.refinenet4")
    for level in (2, 1, 0):
        h, w = pyr[level].shape[2], pyr[level].shape[3]
        path = path[:, :, :h, :w]
        path = _fusion(path, pyr[level], p, f"dense_head.0.scratch.refinenet{level + 1}")
    out = C.conv(path, p, "dense_head.1.conv1", padding=1)
    out = C.resize_bilinear(out, R * C.PATCH, Cc * C.PATCH)
    return C.conv(F.relu(C.conv(out, p, "dense_head.1.conv2.0", padding=1)), p, "dense_head.1.conv2.2")


def pose_head(p, spatial):
    """mapanything-rs/src/heads.rs:80-99. spatial [V, d, h, w] -> (t [V,3], unit q [V,4])."""
    x = C.conv(spatial, p, "pose_head.proj")
    for blk in range(2):
        r = x
        for k in range(1, 4):
            r = F.relu(C.conv(r, p, f"pose_head.res_conv.{blk}.res_conv{k}"))
        x = x + r
    pooled = x.flatten(2).mean(-1)
    for name in ("more_mlps.0", "more_mlps.2"):
        pooled = F.relu(C.linear(pooled, p, "pose_head." + name))
    quat = C.linear(pooled, p, "pose_head.fc_rot")
    norm = quat.pow(2).sum(-1, keepdim=True).sqrt().clamp(min=QUAT_MIN_NORM)
    return C.linear(pooled, p, "pose_head.fc_t"), quat / norm


def scale_head(p, token):
    """mapanything-rs/src/heads.rs:122-129"""
    x = C.linear(token, p, "scale_head.proj")
    for layer in range(2):
        x = F.relu(C.linear(x, p, f"scale_head.mlp.{layer}.0"))
    return torch.exp(C.linear(x, p, "scale_head.output_proj")).clamp(min=MIN_SCALE).flatten()


def dense_output(raw, scale):
    """mapanything-rs/src/model.rs:148-172 for [V, 6, H, W] raw maps."""
    rays = raw[:, 0:3]
    norm = rays.pow(2).sum(1, keepdim=True).sqrt().clamp(min=RAY_MIN_NORM)
    depth = torch.exp(raw[:, 3:4]) * scale
    points = rays / norm * depth
    return points, CONF_MIN + torch.exp(raw[:, 4]), raw[:, 5] > 0


def ray_map(intrinsics, height: int, width: int) -> torch.Tensor:
    """mapanything-rs/src/model.rs:38-54: [3, H, W] unit directions of pinhole rays, pixel
    centres at integer coordinates, computed in f64 and stored as f32. intrinsics =
    (fx, fy, cx, cy)."""
    fx, fy, cx, cy = (float(v) for v in intrinsics)
    xs = (torch.arange(width, dtype=torch.float64) - cx) / fx
    ys = (torch.arange(height, dtype=torch.float64) - cy) / fy
    d = torch.stack([xs[None, :].expand(height, width), ys[:, None].expand(height, width),
                     torch.ones(height, width, dtype=torch.float64)])
    return (d / d.norm(dim=0, keepdim=True)).float()


def pixel_unshuffle(x: torch.Tensor, r: int) -> torch.Tensor:
    """mapanything-rs/src/ray_encoder.rs:48-54 (torch's PixelUnshuffle): [B, C, h*r, w*r] ->
    [B, C*r*r, h, w], channel-major, then row, then column within the block."""
    B, Cn, H, W = x.shape
    return x.reshape(B, Cn, H // r, r, W // r, r).permute(0, 1, 3, 5, 2, 4).reshape(B, Cn * r * r, H // r, W // r)


def ray_encoder(p, rays: torch.Tensor) -> torch.Tensor:
    """mapanything-rs/src/ray_encoder.rs:56-86: rays [B, 3, H, W] -> patch features [B, P, dim].
    conv_in 3x3 (588 -> 588), two residual blocks gelu(conv2(gelu(conv1(x))) + shortcut(x))
    (588 -> 768 -> 1024; 3x3, 3x3, 1x1), encoder.2 1x1 (1024 -> dim), LayerNorm eps 1e-6. The
    reference runs it in f32 whatever the model dtype (model.rs:72-73)."""
    q = "ray_dirs_encoder."
    x = C.conv(pixel_unshuffle(rays, C.PATCH), p, q + "conv_in", padding=1)
    for i in range(2):
        b = f"{q}encoder.{i}."
        h = C.gelu(C.conv(x, p, b + "conv1", padding=1))
        x = C.gelu(C.conv(h, p, b + "conv2", padding=1) + C.conv(x, p, b + "shortcut"))
    x = C.conv(x, p, q + "encoder.2").flatten(2).transpose(1, 2)
    return C.layer_norm(x, p[q + "norm_layer.weight"], p[q + "norm_layer.bias"], LN_EPS)


def forward(weights, spec, images, dtype=torch.float32, encoder_only=False, taps=None, info_taps=None,
            intrinsics=None, branch_taps=None, info_branch_taps=None) -> dict:
    """mapanything-rs/src/model.rs:86-144. intrinsics: None, or one entry per view, each None
    (unknown camera, model.rs:103) or (fx, fy, cx, cy) (known: the ray encoder's features are
    added to the image patches before the fusion norm, model.rs:97-102)."""
    p = C.to_torch(weights, dtype) if not isinstance(next(iter(weights.values())), torch.Tensor) else weights
    x = torch.as_tensor(np.asarray(images)).to(dtype)
    V, _, H, W = x.shape
    R, Cc = H // C.PATCH, W // C.PATCH
    P = R * Cc
    with torch.no_grad():
        tokens = encoder_forward(p, spec, x, taps, branch_taps)
        if encoder_only:
            return {"encoder_tokens": tokens.float()}
        patches = tokens[:, 1:]
        if intrinsics is not None and any(k is not None for k in intrinsics):
            rdt = torch.float64 if dtype == torch.float64 else torch.float32
            rp = {k: v.to(rdt) for k, v in p.items() if k.startswith("ray_dirs_encoder.")}
            add = torch.zeros_like(patches)
            for v, k in enumerate(intrinsics):
                if k is not None:
                    add[v] = ray_encoder(rp, ray_map(k, H, W)[None].to(rdt))[0].to(patches.dtype)
            patches = patches + add
        fused = C.layer_norm(patches, p["fusion_norm_layer.weight"], p["fusion_norm_layer.bias"], LN_EPS)
        classes = tokens[:, :1]
        info_patches, info_classes = fused, classes
        if spec.has_proj:
            info_patches = C.linear(fused, p, "info_sharing.proj_embed")
            info_classes = C.linear(classes, p, "info_sharing.proj_embed")
        per_view, scale_tok = info_sharing_forward(p, spec, info_patches, info_classes, info_taps, info_branch_taps)
        scale = scale_head(p, scale_tok[None])[0]
        hooks = [fused] + [torch.stack([pv[k] for pv in per_view]) for k in range(3)]
        raw = dpt_forward(p, spec, hooks, R, Cc).float()
        last = hooks[3]
        spatial = last.transpose(1, 2).reshape(V, spec.info_dim, R, Cc)
        trans, quat = pose_head(p, spatial)
        points, conf, mask = dense_output(raw, scale.float())
    return {
        "raw": raw,
        "scale": float(scale),
        "quaternion": quat.float(),
        "translation": (trans.float() * scale.float()),
        "translation_raw": trans.float(),
        "points": points.float(),
        "conf": conf.float(),
        "mask": mask,
        "encoder_tokens": tokens.float(),
    }
