"""CPU oracle, shared pieces — TEST INFRASTRUCTURE ONLY.

A restatement, from the reference's Rust source read as text, of the arithmetic the
feed-forward network path performs. Only `tests/`, `__graft_entry__.smoke()` and the
`cpu_baseline` leg of `bench.py` may import this package, and only as the checker or the
timed CPU baseline: the product (the HIP library) never calls it.

Each function cites the reference file:line it follows. How each one is pinned: the
elementary functions by known-answer tests from the reference's own unit tests, library
routines, closed forms and brute force (tests/test_oracle.py); the composite functions
(transformer block, residual units, fusion blocks and chains, both DPT heads, camera, pose and
scale heads, dense_output, the info-sharing transformer and the MapAnything assembly) by closed
forms under structured weights that a swapped operand or reordered op fails
(tests/test_oracle_composites.py). The reference has no network-level golden vector
(depthanything3-rs/README.md and mapanything-rs/README.md state its numerics are unchecked);
what only candle itself could pin (its gelu_erf approximation, LayerNorm statistic precision,
bf16 rounding points between ops, Metal sdpa) stays "parity unpinned" and the tolerances
absorb it.

Candle op semantics restated here with PyTorch CPU library routines (the un-vendored
candle-core/candle-nn 0.11.0 ops of the reference, Cargo.lock:668-731):
  Conv2d (weight [out,in,kh,kw], zero padding)       -> F.conv2d
  ConvTranspose2d (weight [in,out,kh,kw])            -> F.conv_transpose2d
  Linear (y = x W^T + b)                             -> F.linear
  LayerNorm (biased variance, eps inside the sqrt)   -> F.layer_norm
  softmax_last_dim / sdpa                            -> blockwise softmax(q k^T * scale) v
  gelu_erf                                           -> F.gelu(approximate="none")
  silu / relu / exp                                  -> F.silu / F.relu / torch.exp
  upsample_bilinear2d(h, w, align_corners=true)      -> F.interpolate(bilinear, align_corners=True)
"""
from __future__ import annotations

import math
from typing import List, Sequence, Tuple

import numpy as np
import torch
import torch.nn.functional as F

PATCH = 14
HEAD_DIM = 64
TRAINED_GRID = 37
INTERPOLATE_OFFSET = 0.1     # depthanything3-rs/src/backbone.rs:24
BICUBIC_A = -0.75            # mapanything-rs/src/dinov2.rs:19


# --- bicubic positional-embedding resize: mapanything-rs/src/dinov2.rs:20-76 -------------

def bicubic_weights(t: float) -> List[float]:
    """mapanything-rs/src/dinov2.rs:20-25"""
    a = BICUBIC_A
    near = lambda x: ((a + 2.0) * x - (a + 3.0)) * x * x + 1.0
    far = lambda x: ((a * x - 5.0 * a) * x + 8.0 * a) * x - 4.0 * a
    return [far(t + 1.0), near(t), near(1.0 - t), far(2.0 - t)]


def bicubic_taps(n_in: int, n_out: int, scale: float):
    """mapanything-rs/src/dinov2.rs:29-38"""
    taps = []
    for o in range(n_out):
        src = (o + 0.5) / scale - 0.5
        fl = math.floor(src)
        idx = [min(max(fl + off, 0), n_in - 1) for off in (-1, 0, 1, 2)]
        taps.append((idx, bicubic_weights(src - fl)))
    return taps


def resize_grid(grid: np.ndarray, rows: int, cols: int, out_rows: int, out_cols: int,
                row_scale: float, col_scale: float) -> np.ndarray:
    """mapanything-rs/src/dinov2.rs:42-76: separable bicubic of a [rows, cols, ch] grid in f64,
    columns first, then rows; result rounded to f32."""
    g = np.asarray(grid, dtype=np.float64).reshape(rows, cols, -1)
    ch = g.shape[2]
    horiz = np.zeros((rows, out_cols, ch), np.float64)
    for oc, (idx, w) in enumerate(bicubic_taps(cols, out_cols, col_scale)):
        for i, wt in zip(idx, w):
            horiz[:, oc, :] += wt * g[:, i, :]
    out = np.zeros((out_rows, out_cols, ch), np.float64)
    for orow, (idx, w) in enumerate(bicubic_taps(rows, out_rows, row_scale)):
        for i, wt in zip(idx, w):
            out[orow] += wt * horiz[i]
    return out.astype(np.float32)


def positional_embedding(pos_embed: torch.Tensor, rows: int, cols: int) -> torch.Tensor:
    """depthanything3-rs/src/backbone.rs:94-112 (= mapanything-rs/src/dinov2.rs:107-125):
    [1, 1+rows*cols, d], class slot untouched, grid resized with scale (out+0.1)/37."""
    if (rows, cols) == (TRAINED_GRID, TRAINED_GRID):
        return pos_embed.float()
    d = pos_embed.shape[-1]
    cls = pos_embed[:, :1].float()
    grid = pos_embed[0, 1:].float().numpy()
    scale = lambda o: (o + INTERPOLATE_OFFSET) / TRAINED_GRID
    resized = resize_grid(grid, TRAINED_GRID, TRAINED_GRID, rows, cols, scale(rows), scale(cols))
    return torch.cat([cls, torch.from_numpy(resized).reshape(1, rows * cols, d)], 1)


# --- 2D RoPE: depthanything3-rs/src/rope.rs:26-73 -----------------------------------------

ROPE_BASE = 100.0


def rope_tables(positions: Sequence[Tuple[int, int]]) -> Tuple[torch.Tensor, torch.Tensor]:
    """depthanything3-rs/src/rope.rs:32-54: cos/sin [tokens, 64], angles in f64, stored f32."""
    freqs = [1.0 / ROPE_BASE ** (p / 16.0) for p in range(16)]
    n = len(positions)
    cos = np.zeros((n, HEAD_DIM), np.float32)
    sin = np.zeros((n, HEAD_DIM), np.float32)
    for t, pos in enumerate(positions):
        for axis, coord in enumerate(pos):
            for p in range(16):
                ang = coord * freqs[p]
                for rep in range(2):
                    ch = axis * 32 + rep * 16 + p
                    cos[t, ch] = math.cos(ang)
                    sin[t, ch] = math.sin(ang)
    return torch.from_numpy(cos), torch.from_numpy(sin)


def rotate_pairs(x: torch.Tensor) -> torch.Tensor:
    """depthanything3-rs/src/rope.rs:57-66: per 32-channel axis half [a, b] -> [-b, a]."""
    parts = []
    for axis in range(2):
        a = x[..., axis * 32: axis * 32 + 16]
        b = x[..., axis * 32 + 16: axis * 32 + 32]
        parts += [-b, a]
    return torch.cat(parts, -1)


def rope_apply(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """depthanything3-rs/src/rope.rs:70-73; x [..., tokens, 64]."""
    return x * cos.to(x.dtype) + rotate_pairs(x) * sin.to(x.dtype)


# --- elementary ops ------------------------------------------------------------------------

def layer_norm(x, w, b, eps):
    return F.layer_norm(x, (x.shape[-1],), w, b, eps)


def linear(x, p, name):
    return F.linear(x, p[name + ".weight"], p.get(name + ".bias"))


def conv(x, p, name, padding=0, stride=1):
    return F.conv2d(x, p[name + ".weight"], p.get(name + ".bias"), stride=stride, padding=padding)


def conv_t(x, p, name, stride):
    return F.conv_transpose2d(x, p[name + ".weight"], p[name + ".bias"], stride=stride)


def resize_bilinear(x, rows, cols):
    """upsample_bilinear2d(rows, cols, align_corners=true): depthanything3-rs/src/dpt.rs:39-41"""
    return F.interpolate(x, size=(rows, cols), mode="bilinear", align_corners=True)


def split_heads(x):
    """[S, L, h*64] -> [S, h, L, 64]: depthanything3-rs/src/vit_block.rs:34-40"""
    s, l, d = x.shape
    return x.reshape(s, l, d // HEAD_DIM, HEAD_DIM).transpose(1, 2)


def merge_heads(x):
    """[S, h, L, 64] -> [S, L, h*64]: depthanything3-rs/src/vit_block.rs:43-46"""
    s, h, l, e = x.shape
    return x.transpose(1, 2).reshape(s, l, h * e)


def attention(q, k, v, chunk: int = 2048):
    """softmax(q k^T / sqrt(64)) v, no mask (depthanything3-rs/src/vit_block.rs:49-67,
    mapanything-rs/src/vit_block.rs:29-38), computed per query chunk so the score matrix of a
    long global sequence is never held whole."""
    scale = 1.0 / math.sqrt(HEAD_DIM)
    out = torch.empty_like(q)
    for s0 in range(0, q.shape[-2], chunk):
        sc = torch.matmul(q[..., s0:s0 + chunk, :], k.transpose(-1, -2)) * scale
        out[..., s0:s0 + chunk, :] = torch.matmul(torch.softmax(sc, -1), v)
    return out


def gelu(x):
    return F.gelu(x, approximate="none")


def feed_forward(x, p, name, swiglu: bool):
    """GELU MLP (depthanything3-rs/src/vit_block.rs:70-79) or SwiGLU
    (mapanything-rs/src/vit_block.rs:48-71: [x1, x2] = w12(x) halves, w3(silu(x1) * x2))."""
    if swiglu:
        x12 = linear(x, p, name + ".w12")
        h = x12.shape[-1] // 2
        return linear(F.silu(x12[..., :h]) * x12[..., h:], p, name + ".w3")
    return linear(gelu(linear(x, p, name + ".fc1")), p, name + ".fc2")


def vit_block(x, p, name, swiglu: bool, block_eps: float, qk_norm: bool = False,
              rope=None, taps=None):
    """Pre-norm block: depthanything3-rs/src/vit_block.rs:149-167 (qk-norm eps 1e-5 and RoPE
    when given) and mapanything-rs/src/vit_block.rs:97-107 (neither). `x`: [S, L, d]."""
    d = x.shape[-1]
    qkv = linear(layer_norm(x, p[name + ".norm1.weight"], p[name + ".norm1.bias"], block_eps), p, name + ".attn.qkv")
    q = split_heads(qkv[..., :d])
    k = split_heads(qkv[..., d:2 * d])
    v = split_heads(qkv[..., 2 * d:])
    if qk_norm:
        q = layer_norm(q, p[name + ".attn.q_norm.weight"], p[name + ".attn.q_norm.bias"], 1e-5)
        k = layer_norm(k, p[name + ".attn.k_norm.weight"], p[name + ".attn.k_norm.bias"], 1e-5)
    if rope is not None:
        q = rope_apply(q, *rope)
        k = rope_apply(k, *rope)
    attended = linear(merge_heads(attention(q, k, v)), p, name + ".attn.proj")
    if taps is not None:
        taps.append(("attn", attended))
    x = x + attended * p[name + ".ls1.gamma"]
    mlp = feed_forward(layer_norm(x, p[name + ".norm2.weight"], p[name + ".norm2.bias"], block_eps),
                       p, name + ".mlp", swiglu)
    if taps is not None:
        taps.append(("mlp", mlp))
    return x + mlp * p[name + ".ls2.gamma"]


def to_torch(weights: dict, dtype=torch.float32) -> dict:
    return {k: torch.as_tensor(np.asarray(v)).to(dtype) for k, v in weights.items()}


IMAGENET_MEAN = np.array([0.485, 0.456, 0.406], np.float32)   # mapanything-rs/src/image_input.rs:113
IMAGENET_STD = np.array([0.229, 0.224, 0.225], np.float32)    # mapanything-rs/src/image_input.rs:114
FOREGROUND_MIN_ALPHA = 128                                      # mapanything-rs/src/image_input.rs:22


def to_model_input(rgba: np.ndarray):
    """mapanything-rs/src/image_input.rs:195-216 for [V, H, W, 4] u8: f32 images [V, 3, H, W] =
    ((x * (1/255) + 0) - mean) / std in f32, in candle's op order (affine, broadcast_sub,
    broadcast_div), and foreground = alpha >= 128."""
    x = np.asarray(rgba, np.uint8)
    rgb = x[..., :3].astype(np.float32).transpose(0, 3, 1, 2)
    v = rgb * np.float32(1.0 / 255.0) + np.float32(0.0)
    v = (v - IMAGENET_MEAN[None, :, None, None]) / IMAGENET_STD[None, :, None, None]
    return v.astype(np.float32), x[..., 3] >= FOREGROUND_MIN_ALPHA
