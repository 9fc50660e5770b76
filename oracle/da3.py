"""CPU oracle for Depth Anything 3 — TEST INFRASTRUCTURE ONLY (see oracle/common.py).

Restates depthanything3-rs/src/{model,backbone,vit_block,rope,reference_view,dpt,uv_embed,
camera_head}.rs in torch-CPU float32 (or float64).
"""
from __future__ import annotations

import math
from typing import Dict, List, Sequence

import numpy as np
import torch
import torch.nn.functional as F

from . import common as C

BLOCK_NORM_EPS = 1e-6         # depthanything3-rs/src/vit_block.rs:15
TORCH_LN_EPS = 1e-5           # depthanything3-rs/src/vit_block.rs:17
CONF_MIN = 1.0                # depthanything3-rs/src/model.rs:21
MIN_VIEWS_FOR_SELECTION = 3   # depthanything3-rs/src/reference_view.rs:9
SCALE_EPS = 1e-8              # depthanything3-rs/src/reference_view.rs:11
REF_FIRST, REF_MIDDLE, REF_SADDLE = 0, 1, 2


# --- reference view: depthanything3-rs/src/reference_view.rs -------------------------------

def select_reference_view(class_tokens: np.ndarray, strategy: int) -> int:
    """depthanything3-rs/src/reference_view.rs:38-80 (f64 arithmetic, first minimum)."""
    views = len(class_tokens)
    if views < MIN_VIEWS_FOR_SELECTION:
        return 0
    if strategy == REF_FIRST:
        return 0
    if strategy == REF_MIDDLE:
        return views // 2
    tok = [np.asarray(t, np.float32).astype(np.float64) for t in class_tokens]
    norms = [math.sqrt(sum(v * v for v in t)) for t in tok]
    unit = [t / n for t, n in zip(tok, norms)]
    sim = [sum(float(np.dot(unit[i], unit[j])) for j in range(views) if j != i) / (views - 1)
           for i in range(views)]

    def variance(u):
        m = float(np.sum(u)) / len(u)
        return float(np.sum((u - m) ** 2)) / (len(u) - 1)

    var = [variance(u) for u in unit]

    def mm(vals):
        lo, hi = min(vals), max(vals)
        return [(v - lo) / (hi - lo + SCALE_EPS) for v in vals]

    s, n, va = mm(sim), mm(norms), mm(var)
    bal = [abs(s[i] - 0.5) + abs(n[i] - 0.5) + abs(va[i] - 0.5) for i in range(views)]
    best = 0
    for i, b in enumerate(bal):
        if b < bal[best]:
            best = i
    return best


def order_with_reference_first(views: int, reference: int) -> List[int]:
    """depthanything3-rs/src/reference_view.rs:84-89"""
    return [reference] + [v for v in range(views) if v != reference]


def positions_of_views(order: Sequence[int]) -> List[int]:
    """depthanything3-rs/src/reference_view.rs:92-99"""
    pos = [None] * len(order)
    for p, v in enumerate(order):
        pos[v] = p
    return pos


def rope_positions(rows: int, cols: int, across_views: bool):
    """depthanything3-rs/src/backbone.rs:53-65"""
    out = [(0, 0)]
    for r in range(rows):
        for c in range(cols):
            out.append((1, 1) if across_views else (r + 1, c + 1))
    return out


# --- uv embedding: depthanything3-rs/src/uv_embed.rs:14-53 ---------------------------------

def uv_embedding(channels: int, rows: int, cols: int, aspect: float) -> torch.Tensor:
    """[1, channels, rows, cols] f32: u (column) in channels [0, C/2), v (row) in [C/2, C);
    each half C/4 sines then C/4 cosines of coord * 100^(-k/(C/4)), times 0.1."""
    assert channels % 4 == 0
    diag = math.sqrt(aspect * aspect + 1.0)
    span = (aspect / diag, 1.0 / diag)

    def coord(i, n, axis):
        edge = span[axis] * (n - 1.0) / n
        return -edge if n == 1 else -edge + 2.0 * edge * i / (n - 1.0)

    half = channels // 2
    q = half // 2
    emb = np.zeros((channels, rows, cols), np.float32)
    fr = np.array([100.0 ** (k / q) for k in range(q)], np.float64)
    cu = np.array([coord(c, cols, 0) for c in range(cols)], np.float64)
    rv = np.array([coord(r, rows, 1) for r in range(rows)], np.float64)
    au = cu[None, :] / fr[:, None]                                      # [q, cols]
    av = rv[None, :] / fr[:, None]                                      # [q, rows]
    emb[0:q] = (np.sin(au).astype(np.float32) * np.float32(0.1))[:, None, :]
    emb[q:half] = (np.cos(au).astype(np.float32) * np.float32(0.1))[:, None, :]
    emb[half:half + q] = (np.sin(av).astype(np.float32) * np.float32(0.1))[:, :, None]
    emb[half + q:] = (np.cos(av).astype(np.float32) * np.float32(0.1))[:, :, None]
    return torch.from_numpy(emb)[None]


# --- backbone: depthanything3-rs/src/backbone.rs:128-196 ----------------------------------

def backbone_forward(p: Dict[str, torch.Tensor], spec, images: torch.Tensor, strategy: int,
                     force_reference: int = None, taps: list = None, branch_taps: list = None):
    V, _, H, W = images.shape
    assert H % C.PATCH == 0 and W % C.PATCH == 0
    R, Cc = H // C.PATCH, W // C.PATCH
    n = 1 + R * Cc
    d = spec.dim
    b = "model.backbone.pretrained"
    dt = images.dtype
    patches = C.conv(images, p, b + ".patch_embed.proj", stride=C.PATCH).flatten(2).transpose(1, 2)
    pos = C.positional_embedding(p[b + ".pos_embed"], R, Cc).to(dt)
    cls = p[b + ".cls_token"].expand(V, 1, d)
    xs = torch.cat([cls, patches], 1) + pos
    within_rope = C.rope_tables(rope_positions(R, Cc, False))
    across_rope = C.rope_tables(rope_positions(R, Cc, True) * V)
    order = list(range(V))
    reference = 0
    within = xs
    layers, camera_tokens = [], None
    swiglu = spec.ffn == 1
    for i in range(spec.depth):
        name = f"{b}.blocks.{i}"
        if i + 1 == spec.alt_start and V >= MIN_VIEWS_FOR_SELECTION:
            reference = select_reference_view(xs[:, 0].float().numpy(), strategy)
            if force_reference is not None:
                reference = force_reference
            order = order_with_reference_first(V, reference)
            xs = xs[order]
        if i == spec.alt_start:
            cam = p[b + ".camera_token"]
            cams = torch.cat([cam[:, 0:1]] + [cam[:, 1:2]] * (V - 1), 0)
            xs = torch.cat([cams, xs[:, 1:]], 1)
        across = i >= spec.alt_start and i % 2 == 1
        qk = i >= spec.alt_start
        bt = [] if branch_taps is not None else None
        if across:
            xs = C.vit_block(xs.reshape(1, V * n, d), p, name, swiglu, BLOCK_NORM_EPS, qk, across_rope, bt).reshape(V, n, d)
        else:
            xs = C.vit_block(xs, p, name, swiglu, BLOCK_NORM_EPS, qk, within_rope if qk else None, bt)
            within = xs
        restore = positions_of_views(order)
        if taps is not None:
            taps.append(xs[restore].clone())
        if branch_taps is not None:
            branch_taps.append([t[1].reshape(V, n, d)[restore].clone() for t in bt])
        if i in spec.out_layers:
            out = torch.cat([within, xs], -1)
            if order != list(range(V)):
                out = out[restore]
            camera_tokens = out[:, 0].contiguous()
            w_part = out[..., :d]
            a_part = C.layer_norm(out[..., d:], p[b + ".norm.weight"], p[b + ".norm.bias"], TORCH_LN_EPS)
            layers.append(torch.cat([w_part, a_part], -1)[:, 1:])
    return layers, camera_tokens, reference


# --- dense head: depthanything3-rs/src/dpt.rs ---------------------------------------------

def _rcu(x, p, name):
    """dpt.rs:104-110: conv2(relu(conv1(relu(x)))) + x"""
    out = C.conv(F.relu(x), p, name + ".conv1", padding=1)
    out = C.conv(F.relu(out), p, name + ".conv2", padding=1)
    return out + x


def _fusion(x, skip, p, name, out_size):
    """dpt.rs:130-137"""
    if skip is not None:
        x = x + _rcu(skip, p, name + ".resConfUnit1")
    return C.conv(C.resize_bilinear(_rcu(x, p, name + ".resConfUnit2"), *out_size), p, name + ".out_conv")


def _chain(pyr, p, scratch, suffix):
    """dpt.rs:156-164"""
    size = lambda t: (t.shape[2], t.shape[3])
    path = _fusion(pyr[3], None, p, f"{scratch}.refinenet4{suffix}", size(pyr[2]))
    for level in (2, 1):
        path = _fusion(path, pyr[level], p, f"{scratch}.refinenet{level + 1}{suffix}", size(pyr[level - 1]))
    r, c = size(pyr[0])
    return _fusion(path, pyr[0], p, f"{scratch}.refinenet1{suffix}", (2 * r, 2 * c))


def _add_uv(x, image_hw):
    _, ch, r, c = x.shape
    return x + uv_embedding(ch, r, c, image_hw[1] / image_hw[0]).to(x.dtype)


def dpt_forward(p, spec, layers, R, Cc):
    """depthanything3-rs/src/dpt.rs:256-300, all views at once (the reference loops views;
    every op is per view)."""
    h = "model.head"
    s = h + ".scratch"
    image_hw = (R * C.PATCH, Cc * C.PATCH)
    pyr = []
    for k, tok in enumerate(layers):
        V, P, D = tok.shape
        sp = C.layer_norm(tok, p[h + ".norm.weight"], p[h + ".norm.bias"], TORCH_LN_EPS)
        sp = sp.transpose(1, 2).reshape(V, D, R, Cc)
        x = _add_uv(C.conv(sp, p, f"{h}.projects.{k}"), image_hw)
        if k == 0:
            x = C.conv_t(x, p, h + ".resize_layers.0", 4)
        elif k == 1:
            x = C.conv_t(x, p, h + ".resize_layers.1", 2)
        elif k == 3:
            x = C.conv(x, p, h + ".resize_layers.3", padding=1, stride=2)
        pyr.append(C.conv(x, p, f"{s}.layer{k + 1}_rn", padding=1))
    fused = C.conv(_chain(pyr, p, s, ""), p, s + ".output_conv1", padding=1)
    fused = _add_uv(C.resize_bilinear(fused, *image_hw), image_hw)
    depth_logits = C.conv(F.relu(C.conv(fused, p, s + ".output_conv2.0", padding=1)), p, s + ".output_conv2.2")
    rays = _chain(pyr, p, s, "_aux")
    for i in range(5):
        rays = C.conv(rays, p, f"{s}.output_conv1_aux.3.{i}", padding=1)
    rays = C.conv(_add_uv(rays, image_hw), p, s + ".output_conv2_aux.3.0", padding=1)
    rays = C.layer_norm(rays.permute(0, 2, 3, 1), None, None, TORCH_LN_EPS).permute(0, 3, 1, 2)
    ray_logits = C.conv(F.relu(rays), p, s + ".output_conv2_aux.3.5")
    return depth_logits, ray_logits


def camera_head(p, camera_tokens):
    """depthanything3-rs/src/camera_head.rs:81-91 -> [V, 9] (t 3, quaternion xyzw 4, fov 2)."""
    c = "model.cam_dec"
    x = camera_tokens
    for name in ("backbone.0", "backbone.2"):
        x = F.relu(C.linear(x, p, f"{c}.{name}"))
    x = x if x.dtype == torch.float64 else x.float()   # output layers in f32 (camera_head.rs:67-68)
    return torch.cat([C.linear(x, p, c + ".fc_t"), C.linear(x, p, c + ".fc_qvec"),
                      F.relu(C.linear(x, p, c + ".fc_fov.0"))], 1)


def forward_raw(weights, spec, images, strategy: int = REF_SADDLE, dtype=torch.float32,
                force_reference: int = None, taps: list = None, branch_taps: list = None) -> dict:
    """depthanything3-rs/src/model.rs:105-123. `weights`: name -> array; `images` [V,3,H,W]."""
    p = C.to_torch(weights, dtype) if not isinstance(next(iter(weights.values())), torch.Tensor) else weights
    x = torch.as_tensor(np.asarray(images)).to(dtype)
    V, _, H, W = x.shape
    R, Cc = H // C.PATCH, W // C.PATCH
    with torch.no_grad():
        layers, cam_tokens, ref = backbone_forward(p, spec, x, strategy, force_reference, taps, branch_taps)
        depth_logits, ray_logits = dpt_forward(p, spec, layers, R, Cc)
        pose = camera_head(p, cam_tokens)
        logits = depth_logits.float()
    return {
        "depth": torch.exp(logits[:, 0]),
        "depth_conf": torch.exp(logits[:, 1]) + CONF_MIN,
        "ray_logits": ray_logits.float(),
        "pose_encoding": pose.float(),
        "camera_tokens": cam_tokens.float(),
        "reference_view": ref,
        "layers": [l.float() for l in layers],
    }


# --- camera estimate: depthanything3-rs/src/camera_head.rs:28-53 --------------------------

def quaternion_to_rotation(qx, qy, qz, qw) -> np.ndarray:
    """nalgebra UnitQuaternion::from_quaternion(Quaternion::new(w, x, y, z)) normalises, then
    the standard rotation matrix."""
    n = math.sqrt(qx * qx + qy * qy + qz * qz + qw * qw)
    x, y, z, w = qx / n, qy / n, qz / n, qw / n
    return np.array([
        [1 - 2 * (y * y + z * z), 2 * (x * y - z * w), 2 * (x * z + y * w)],
        [2 * (x * y + z * w), 1 - 2 * (x * x + z * z), 2 * (y * z - x * w)],
        [2 * (x * z - y * w), 2 * (y * z + x * w), 1 - 2 * (x * x + y * y)],
    ])


def focal(fov_h: float, fov_w: float, height: int, width: int):
    """camera_head.rs:42-48"""
    return (width / 2.0 / max(math.tan(fov_w / 2.0), 1e-6),
            height / 2.0 / max(math.tan(fov_h / 2.0), 1e-6))
