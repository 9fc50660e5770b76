"""Closed-form pins of the oracle's composite functions (CPU, float64).

Each test gives a composite (a transformer block, a residual unit, a fusion chain, a whole DPT
head, a pose/scale/camera head, the info-sharing transformer, dense_output) structured weights
(zeros, identities, channel selections, distinct scalars) under which the reference's op order
reduces to a short closed form, computed here from first principles or from primitives pinned
in test_oracle.py (LayerNorm, bilinear align_corners, uv embedding). The weights are chosen so
that a plausible slip fails: swapped q/k/v slices, q- and k-norm exchanged, RoPE on v, a ReLU
moved inside a residual unit, resConfUnit1/2 exchanged, a crop after instead of before the
fusion, refinenet levels or hook indices off by one, a norm applied to the wrong tensor, a
missing or extra activation. Reference files are cited per test.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import common as C
from oracle import da3 as OD
from oracle import mapanything as OM
from splathip import specs, synth

D64 = torch.float64


def ln(x, eps):
    """LayerNorm without affine from its definition: biased variance, eps inside the sqrt."""
    m = x.mean(-1, keepdim=True)
    v = ((x - m) ** 2).mean(-1, keepdim=True)
    return (x - m) / torch.sqrt(v + eps)


def gelu_exact(x):
    return 0.5 * x * (1 + torch.erf(x / math.sqrt(2)))


def sel(rows, cols, scale=1.0):
    """[rows, cols] matrix with `scale` on the leading diagonal (a channel selection/embedding)."""
    m = torch.zeros(rows, cols, dtype=D64)
    k = min(rows, cols)
    m[range(k), range(k)] = scale
    return m


def conv_center(cout, cin, scale=1.0):
    """3x3 kernel whose centre tap is sel(cout, cin, scale): a per-pixel channel map."""
    w = torch.zeros(cout, cin, 3, 3, dtype=D64)
    w[:, :, 1, 1] = sel(cout, cin, scale)
    return w


def conv1x1(cout, cin, scale=1.0):
    return sel(cout, cin, scale)[:, :, None, None].clone()


def convt_nearest(c, s):
    """ConvTranspose2d(c, c, kernel = stride = s) weights that replicate each pixel s x s."""
    w = torch.zeros(c, c, s, s, dtype=D64)
    for i in range(c):
        w[i, i] = 1.0
    return w


def nearest_up(x, s):
    return x.repeat_interleave(s, 2).repeat_interleave(s, 3)


def up_ac(x, h, w):
    """upsample_bilinear2d(align_corners=true): the library routine pinned in test_oracle.py."""
    return F.interpolate(x, size=(h, w), mode="bilinear", align_corners=True)


def zeros_like_params(p):
    return {k: torch.zeros_like(v) for k, v in p.items()}


def set_identity_rcu(p, name, f):
    """conv2(relu(conv1(relu(x)))) + x with conv1 = -I, conv2 = I, zero biases is x: the first
    ReLU makes conv1's output <= 0, the second zeroes it."""
    p[name + ".conv1.weight"] = conv_center(f, f, -1.0)
    p[name + ".conv1.bias"] = torch.zeros(f, dtype=D64)
    p[name + ".conv2.weight"] = conv_center(f, f, 1.0)
    p[name + ".conv2.bias"] = torch.zeros(f, dtype=D64)


def rng_t(g, *shape, scale=1.0):
    return torch.randn(*shape, generator=g, dtype=D64) * scale


# --- transformer block: depthanything3-rs/src/vit_block.rs:149-167, mapanything-rs/src/vit_block.rs:97-107

def _block_params(g, d, hidden, name="b"):
    p = {}
    p[name + ".norm1.weight"], p[name + ".norm1.bias"] = torch.ones(d, dtype=D64), torch.zeros(d, dtype=D64)
    p[name + ".norm2.weight"], p[name + ".norm2.bias"] = 1 + rng_t(g, d, scale=0.2), rng_t(g, d, scale=0.2)
    p[name + ".attn.qkv.weight"] = torch.zeros(3 * d, d, dtype=D64)
    p[name + ".attn.qkv.bias"] = torch.zeros(3 * d, dtype=D64)
    p[name + ".attn.proj.weight"], p[name + ".attn.proj.bias"] = rng_t(g, d, d, scale=0.2), rng_t(g, d)
    p[name + ".ls1.gamma"], p[name + ".ls2.gamma"] = rng_t(g, d), rng_t(g, d)
    fc1 = torch.zeros(hidden, d, dtype=D64)
    fc1[:d] = torch.eye(d, dtype=D64)
    p[name + ".mlp.fc1.weight"], p[name + ".mlp.fc1.bias"] = fc1, torch.zeros(hidden, dtype=D64)
    M = rng_t(g, d, d, scale=0.2)
    fc2 = torch.zeros(d, hidden, dtype=D64)
    fc2[:, :d] = M
    p[name + ".mlp.fc2.weight"], p[name + ".mlp.fc2.bias"] = fc2, rng_t(g, d)
    return p, M


def test_block_value_slice_uniform_attention_layerscale_and_norm2_order():
    """q = k = 0 (their weight rows and biases zero) makes every score 0, so attention is the
    mean of v over the sequence; v = A LN1(x) + bv comes from the third column block of qkv.
    Then x1 = x + g1 (P mean(v) + bp) and out = x1 + g2 (M gelu(LN2(x1)) + bf), LN2 on x1 (the
    stream after the attention residual) and the exact GELU between fc1 = [I; 0] and
    fc2 = [M, 0]."""
    g = torch.Generator().manual_seed(0)
    S, L, d = 2, 5, 128
    p, M = _block_params(g, d, 4 * d)
    A, bv = rng_t(g, d, d, scale=0.3), rng_t(g, d)
    p["b.attn.qkv.weight"][2 * d:] = A
    p["b.attn.qkv.bias"][2 * d:] = bv
    w2, b2 = p["b.norm2.weight"], p["b.norm2.bias"]
    x = rng_t(g, S, L, d)
    taps = []
    out = C.vit_block(x, p, "b", False, 1e-6, taps=taps)
    v = ln(x, 1e-6) @ A.T + bv
    att = v.mean(1, keepdim=True).expand(S, L, d) @ p["b.attn.proj.weight"].T + p["b.attn.proj.bias"]
    x1 = x + p["b.ls1.gamma"] * att
    mlp = gelu_exact(ln(x1, 1e-6) * w2 + b2) @ M.T + p["b.mlp.fc2.bias"]
    assert torch.allclose(taps[0][1], att, atol=1e-12) and torch.allclose(taps[1][1], mlp, atol=1e-12)
    assert torch.allclose(out, x1 + p["b.ls2.gamma"] * mlp, atol=1e-12)


@pytest.mark.parametrize("zero", ["k", "q"])
def test_block_query_and_key_slices(zero):
    """With the key block of qkv (rows d..2d-1) zero, or the query block (rows 0..d-1) zero,
    every score is 0 and attention is the mean of v; reading q or k from any other column
    block of qkv gives two non-zero projections and non-uniform weights."""
    g = torch.Generator().manual_seed(20)
    S, L, d = 2, 6, 128
    p, _ = _block_params(g, d, 4 * d)
    W = rng_t(g, 3 * d, d, scale=0.5)
    W[(d if zero == "k" else 0):(2 * d if zero == "k" else d)] = 0.0
    p["b.attn.qkv.weight"] = W
    x = rng_t(g, S, L, d)
    taps = []
    C.vit_block(x, p, "b", False, 1e-6, taps=taps)
    v = ln(x, 1e-6) @ W[2 * d:].T
    att = v.mean(1, keepdim=True).expand(S, L, d) @ p["b.attn.proj.weight"].T + p["b.attn.proj.bias"]
    assert torch.allclose(taps[0][1], att, atol=1e-12)


def test_block_query_and_key_roles_and_qk_norms():
    """q-norm with weight 0 and bias bq makes every query bq; k-norm plain makes k_j = LN(k_j).
    Every query then sees the same softmax over the keys, p = softmax(LN(K) bq / 8), so every
    row of the attention output is sum_j p_j v_j (one head of 64). Exchanging the q and k
    slices, or the two norms (keys all equal -> uniform weights), changes the rows."""
    g = torch.Generator().manual_seed(1)
    S, L, d = 1, 7, 64
    p, _ = _block_params(g, d, 4 * d)
    Wq, Wk, Wv = (rng_t(g, d, d, scale=0.5) for _ in range(3))
    p["b.attn.qkv.weight"] = torch.cat([Wq, Wk, Wv])
    p["b.attn.qkv.bias"] = rng_t(g, 3 * d, scale=0.1)
    bq = rng_t(g, 64, scale=2.0)
    p["b.attn.q_norm.weight"], p["b.attn.q_norm.bias"] = torch.zeros(64, dtype=D64), bq
    p["b.attn.k_norm.weight"], p["b.attn.k_norm.bias"] = torch.ones(64, dtype=D64), torch.zeros(64, dtype=D64)
    x = rng_t(g, S, L, d)
    taps = []
    C.vit_block(x, p, "b", False, 1e-6, qk_norm=True, taps=taps)
    h = ln(x, 1e-6)
    k = ln(h @ Wk.T + p["b.attn.qkv.bias"][d:2 * d], 1e-5)
    v = h @ Wv.T + p["b.attn.qkv.bias"][2 * d:]
    w = torch.softmax(k[0] @ bq / 8.0, 0)
    att = (w[:, None] * v[0]).sum(0)
    want = att @ p["b.attn.proj.weight"].T + p["b.attn.proj.bias"]
    assert torch.allclose(taps[0][1][0], want.expand(L, d), atol=1e-12)
    assert float(w.max() - w.min()) > 0.05   # the weights are far from uniform


def test_block_rope_at_one_shared_position_leaves_attention_unchanged():
    """RoPE rotates q and k (rope.rs:70-73, after the norm). When every token sits at the same
    position both are rotated by the same orthogonal map, so every score, and the block's
    output, is unchanged; RoPE applied to v (or to q only) would change it."""
    g = torch.Generator().manual_seed(2)
    S, L, d = 2, 6, 128
    p, _ = _block_params(g, d, 4 * d)
    p["b.attn.qkv.weight"] = rng_t(g, 3 * d, d, scale=0.3)
    for n in ("q_norm", "k_norm"):
        p[f"b.attn.{n}.weight"], p[f"b.attn.{n}.bias"] = 1 + rng_t(g, 64, scale=0.1), rng_t(g, 64, scale=0.1)
    x = rng_t(g, S, L, d)
    plain = C.vit_block(x, p, "b", False, 1e-6, qk_norm=True)
    rope = C.rope_tables([(3, 7)] * L)
    rotated = C.vit_block(x, p, "b", False, 1e-6, qk_norm=True, rope=rope)
    # the tables hold f32 cos/sin (rope.rs:32-54), orthogonal to ~1e-7
    same = float((plain - rotated).abs().max() / plain.abs().max())
    assert same < 1e-6, same
    # distinct positions do change it (the rotation is applied at all)
    moved = C.vit_block(x, p, "b", False, 1e-6, qk_norm=True, rope=C.rope_tables([(r, r + 1) for r in range(L)]))
    assert float((plain - moved).abs().max() / plain.abs().max()) > 1e3 * max(same, 1e-9)


def test_swiglu_gates_the_first_half_with_the_second():
    """mapanything-rs/src/vit_block.rs:64-70: [x1, x2] = w12(x) by halves, w3(silu(x1) * x2)."""
    g = torch.Generator().manual_seed(3)
    d, h = 16, 24
    A, B, W3 = rng_t(g, h, d), rng_t(g, h, d), rng_t(g, d, h)
    b12, b3 = rng_t(g, 2 * h), rng_t(g, d)
    p = {"m.w12.weight": torch.cat([A, B]), "m.w12.bias": b12, "m.w3.weight": W3, "m.w3.bias": b3}
    x = rng_t(g, 3, d)
    x1, x2 = x @ A.T + b12[:h], x @ B.T + b12[h:]
    want = (x1 / (1 + torch.exp(-x1)) * x2) @ W3.T + b3
    assert torch.allclose(C.feed_forward(x, p, "m", True), want, atol=1e-12)


# --- residual units, fusion blocks, chains: depthanything3-rs/src/dpt.rs:104-164,
# mapanything-rs/src/dpt.rs:109-140

@pytest.mark.parametrize("rcu", [OD._rcu, OM._rcu])
def test_residual_unit_relu_placement(rcu):
    """conv2(relu(conv1(relu(x)))) + x with 3x3 centre-tap identities: conv1 = -I, conv2 = I
    gives x (no first ReLU: x + relu(-x); no second: min(x, 0)); conv1 = I, conv2 = -I gives
    min(x, 0) (a ReLU after conv2 instead: x)."""
    g = torch.Generator().manual_seed(4)
    f = 6
    x = rng_t(g, 2, f, 4, 5)
    p = {}
    set_identity_rcu(p, "u", f)
    assert torch.allclose(rcu(x, p, "u"), x, atol=1e-12)
    p["u.conv1.weight"], p["u.conv2.weight"] = conv_center(f, f, 1.0), conv_center(f, f, -1.0)
    assert torch.allclose(rcu(x, p, "u"), torch.clamp(x, max=0), atol=1e-12)


def _fusion_params(name, f, alpha, skip=True):
    p = {}
    if skip:
        set_identity_rcu(p, name + ".resConfUnit1", f)
    p[name + ".resConfUnit2.conv1.weight"] = conv_center(f, f, 1.0)
    p[name + ".resConfUnit2.conv1.bias"] = torch.zeros(f, dtype=D64)
    p[name + ".resConfUnit2.conv2.weight"] = conv_center(f, f, 1.0)
    p[name + ".resConfUnit2.conv2.bias"] = torch.zeros(f, dtype=D64)
    p[name + ".out_conv.weight"] = conv1x1(f, f, alpha)
    p[name + ".out_conv.bias"] = torch.zeros(f, dtype=D64)
    return p


def test_fusion_block_unit_order_da3():
    """RCU1 (here the identity) on the skip, RCU2 (here y -> relu(y) + y) on the sum, resize,
    out_conv (alpha I): alpha * resize(relu(x + s) + x + s). Exchanged units give
    alpha * resize(x + relu(s) + s)."""
    g = torch.Generator().manual_seed(5)
    f = 4
    p = _fusion_params("r", f, 1.5)
    x, s = rng_t(g, 1, f, 3, 4), rng_t(g, 1, f, 3, 4)
    got = OD._fusion(x, s, p, "r", (5, 7))
    y = x + s
    assert torch.allclose(got, 1.5 * up_ac(torch.relu(y) + y, 5, 7), atol=1e-12)


def test_fusion_block_unit_order_mapanything():
    g = torch.Generator().manual_seed(6)
    f = 4
    p = _fusion_params("r", f, 0.5)
    x, s = rng_t(g, 1, f, 3, 4), rng_t(g, 1, f, 3, 4)
    y = x + s
    assert torch.allclose(OM._fusion(x, s, p, "r"), 0.5 * up_ac(torch.relu(y) + y, 6, 8), atol=1e-12)


def _chain_params(prefix, suffix, f, alphas):
    p = {}
    for level in range(1, 5):
        name = f"{prefix}.refinenet{level}{suffix}"
        p.update(_fusion_params(name, f, alphas[level - 1], skip=level < 4))
        set_identity_rcu(p, name + ".resConfUnit2", f)
    return p


def test_da3_chain_levels_sizes_and_names():
    """With identity units and out_conv of refinenet k equal to alpha_k I, the chain is
    a1 R2x(a2 R(a3 R(a4 R(p3 -> p2) + p2 -> p1) + p1 -> p0) + p0) with R the align_corners
    resize to the next finer level's size and R2x to twice the finest (dpt.rs:156-164)."""
    g = torch.Generator().manual_seed(7)
    f = 3
    al = (1.25, 0.75, 1.5, 2.0)
    p = _chain_params("s", "", f, al)
    pyr = [rng_t(g, 1, f, 8, 10), rng_t(g, 1, f, 4, 5), rng_t(g, 1, f, 3, 3), rng_t(g, 1, f, 2, 2)]
    t = al[3] * up_ac(pyr[3], 3, 3)
    t = al[2] * up_ac(t + pyr[2], 4, 5)
    t = al[1] * up_ac(t + pyr[1], 8, 10)
    want = al[0] * up_ac(t + pyr[0], 16, 20)
    assert torch.allclose(OD._chain(pyr, p, "s", ""), want, atol=1e-12)


# --- whole DPT heads with structured weights ------------------------------------------------

def _hook_map(tokens, R, Cc):
    V, P, D = tokens.shape
    return tokens.transpose(1, 2).reshape(V, D, R, Cc)


def _embed(x, cout):
    """First min(C, cout) channels of x, zero channels after: a selection 1x1 / centre tap."""
    V, Cn, H, W = x.shape
    out = torch.zeros(V, cout, H, W, dtype=x.dtype)
    k = min(Cn, cout)
    out[:, :k] = x[:, :k]
    return out


def test_mapanything_dpt_head_closed_form():
    """mapanything-rs/src/dpt.rs:174-199 with structured weights: 1x1 projections that keep the
    first c_h channels, nearest-neighbour transposed convs (x4, x2), a stride-2 centre tap
    (pixel (2r, 2c)), 3x3 centre-tap feature maps, identity residual units and out_conv
    alpha_k I, so each fusion is alpha_k * up2x(path + skip) with the path cropped to the
    skip's size first; then conv1 (first F/2 channels), bilinear to H x W, relu(conv2.0 = I),
    conv2.2 (first 6 channels). A 3 x 5 patch grid makes the 2x map one row and column too
    large, so cropping after the fusion instead of before gives other values."""
    spec = specs.MA_SPECS["tiny"]
    R, Cc, V = 3, 5, 2
    f, dims = spec.dpt_features, spec.dpt_dims
    g = torch.Generator().manual_seed(8)
    hooks = [rng_t(g, V, R * Cc, spec.enc_dim if h == 0 else spec.info_dim) for h in range(4)]
    p = {}
    for h in range(4):
        hp = f"dense_head.0.input_process.{h}"
        din = spec.enc_dim if h == 0 else spec.info_dim
        p[hp + ".0.0.weight"], p[hp + ".0.0.bias"] = conv1x1(dims[h], din), torch.zeros(dims[h], dtype=D64)
        if h in (0, 1):
            s = 4 if h == 0 else 2
            p[hp + ".0.1.weight"], p[hp + ".0.1.bias"] = convt_nearest(dims[h], s), torch.zeros(dims[h], dtype=D64)
        elif h == 3:
            p[hp + ".0.1.weight"], p[hp + ".0.1.bias"] = conv_center(dims[h], dims[h]), torch.zeros(dims[h], dtype=D64)
        p[hp + ".1.weight"] = conv_center(f, dims[h])
    al = (1.5, 0.5, 1.25, 0.75)
    p.update(_chain_params("dense_head.0.scratch", "", f, al))
    p["dense_head.1.conv1.weight"], p["dense_head.1.conv1.bias"] = conv_center(f // 2, f), torch.zeros(f // 2, dtype=D64)
    p["dense_head.1.conv2.0.weight"] = conv_center(f // 2, f // 2)
    p["dense_head.1.conv2.0.bias"] = torch.zeros(f // 2, dtype=D64)
    p["dense_head.1.conv2.2.weight"], p["dense_head.1.conv2.2.bias"] = conv1x1(6, f // 2), torch.zeros(6, dtype=D64)
    got = OM.dpt_forward(p, spec, hooks, R, Cc)

    pyr = []
    for h in range(4):
        x = _embed(_hook_map(hooks[h], R, Cc), dims[h])
        x = nearest_up(x, 4) if h == 0 else nearest_up(x, 2) if h == 1 else x[:, :, ::2, ::2] if h == 3 else x
        pyr.append(_embed(x, f))
    t = al[3] * up_ac(pyr[3], 2 * pyr[3].shape[2], 2 * pyr[3].shape[3])
    for level in (2, 1, 0):
        hh, ww = pyr[level].shape[2:]
        t = al[level] * up_ac(t[:, :, :hh, :ww] + pyr[level], 2 * hh, 2 * ww)
    want = torch.relu(up_ac(_embed(t, f // 2), R * 14, Cc * 14))[:, :6]
    assert got.shape == (V, 6, R * 14, Cc * 14)
    assert torch.allclose(got, want, atol=1e-12)


def test_da3_dual_dpt_head_closed_form():
    """depthanything3-rs/src/dpt.rs:256-300 with structured weights: the head LayerNorm (eps
    1e-5, weight 1, bias 0) on the tokens, projections keeping the first c_k channels, + uv
    (image aspect W/H) after the projection, nearest transposed convs, stride-2 centre tap,
    centre-tap feature maps; depth chain out_convs alpha_k I and ray chain beta_k I with
    identity units; depth: first 32 channels, bilinear to the image, + uv, relu(conv2.0 = I),
    conv2.2 keeps channels 0-1; rays: five centre taps keep the first 32 channels, + uv,
    conv2_aux.3.0 = I, channel LayerNorm without affine (eps 1e-5), relu, 1x1 keeps 7."""
    spec = specs.DA3_VARIANTS["small"]
    R, Cc, V = 3, 4, 1
    f, dims, hin = spec.head_features, spec.head_stage_dims, spec.head_input_dim
    H, W = R * 14, Cc * 14
    g = torch.Generator().manual_seed(9)
    layers = [rng_t(g, V, R * Cc, hin) for _ in range(4)]
    h, s = "model.head", "model.head.scratch"
    p = {h + ".norm.weight": torch.ones(hin, dtype=D64), h + ".norm.bias": torch.zeros(hin, dtype=D64)}
    for k in range(4):
        p[f"{h}.projects.{k}.weight"], p[f"{h}.projects.{k}.bias"] = conv1x1(dims[k], hin), torch.zeros(dims[k], dtype=D64)
        p[f"{s}.layer{k + 1}_rn.weight"] = conv_center(f, dims[k])
    p[h + ".resize_layers.0.weight"], p[h + ".resize_layers.0.bias"] = convt_nearest(dims[0], 4), torch.zeros(dims[0], dtype=D64)
    p[h + ".resize_layers.1.weight"], p[h + ".resize_layers.1.bias"] = convt_nearest(dims[1], 2), torch.zeros(dims[1], dtype=D64)
    p[h + ".resize_layers.3.weight"], p[h + ".resize_layers.3.bias"] = conv_center(dims[3], dims[3]), torch.zeros(dims[3], dtype=D64)
    al, be = (1.5, 0.5, 1.25, 0.75), (0.25, 2.0, 0.5, 1.75)
    p.update(_chain_params(s, "", f, al))
    p.update(_chain_params(s, "_aux", f, be))
    z = lambda n: torch.zeros(n, dtype=D64)
    p[s + ".output_conv1.weight"], p[s + ".output_conv1.bias"] = conv_center(f // 2, f), z(f // 2)
    p[s + ".output_conv2.0.weight"], p[s + ".output_conv2.0.bias"] = conv_center(32, f // 2), z(32)
    p[s + ".output_conv2.2.weight"], p[s + ".output_conv2.2.bias"] = conv1x1(2, 32), z(2)
    for i in range(5):
        cin, cout = (f, f // 2) if i % 2 == 0 else (f // 2, f)
        p[f"{s}.output_conv1_aux.3.{i}.weight"], p[f"{s}.output_conv1_aux.3.{i}.bias"] = conv_center(cout, cin), z(cout)
    p[s + ".output_conv2_aux.3.0.weight"], p[s + ".output_conv2_aux.3.0.bias"] = conv_center(32, f // 2), z(32)
    p[s + ".output_conv2_aux.3.5.weight"], p[s + ".output_conv2_aux.3.5.bias"] = conv1x1(7, 32), z(7)
    depth, rays = OD.dpt_forward(p, spec, layers, R, Cc)

    uv = lambda ch, r, c: OD.uv_embedding(ch, r, c, W / H).to(D64)
    pyr = []
    for k in range(4):
        x = _embed(_hook_map(ln(layers[k], 1e-5), R, Cc), dims[k]) + uv(dims[k], R, Cc)
        x = nearest_up(x, 4) if k == 0 else nearest_up(x, 2) if k == 1 else x[:, :, ::2, ::2] if k == 3 else x
        pyr.append(_embed(x, f))

    def chain(a):
        t = a[3] * up_ac(pyr[3], *pyr[2].shape[2:])
        t = a[2] * up_ac(t + pyr[2], *pyr[1].shape[2:])
        t = a[1] * up_ac(t + pyr[1], *pyr[0].shape[2:])
        return a[0] * up_ac(t + pyr[0], 2 * pyr[0].shape[2], 2 * pyr[0].shape[3])

    d = up_ac(_embed(chain(al), f // 2), H, W) + uv(f // 2, H, W)
    assert torch.allclose(depth, torch.relu(d)[:, :2], atol=1e-12)
    r = _embed(chain(be), f // 2)
    r = r + uv(f // 2, *r.shape[2:])
    r = ln(r.permute(0, 2, 3, 1), 1e-5).permute(0, 3, 1, 2)
    assert rays.shape == (V, 7, 8 * R, 8 * Cc)
    assert torch.allclose(rays, torch.relu(r)[:, :7], atol=1e-12)


# --- heads ----------------------------------------------------------------------------------

def test_da3_camera_head_order_and_activations():
    """depthanything3-rs/src/camera_head.rs:81-91 with hidden layers I: x = relu(relu(tok));
    fc_t, fc_qvec select channels 0-2 and 3-6, fc_fov.0 selects 7-8 negated (ReLU -> 0) or
    as is; output [t, q, relu(fov)]."""
    n = 12
    g = torch.Generator().manual_seed(10)
    tok = rng_t(g, 3, n)
    c = "model.cam_dec"
    p = {c + ".backbone.0.weight": torch.eye(n, dtype=D64), c + ".backbone.0.bias": torch.zeros(n, dtype=D64),
         c + ".backbone.2.weight": torch.eye(n, dtype=D64), c + ".backbone.2.bias": torch.zeros(n, dtype=D64)}
    rows = lambda idx, sgn=1.0: sgn * torch.eye(n, dtype=D64)[idx]
    p[c + ".fc_t.weight"], p[c + ".fc_t.bias"] = rows([0, 1, 2]), torch.zeros(3, dtype=D64)
    p[c + ".fc_qvec.weight"], p[c + ".fc_qvec.bias"] = rows([3, 4, 5, 6]), torch.zeros(4, dtype=D64)
    p[c + ".fc_fov.0.weight"], p[c + ".fc_fov.0.bias"] = rows([7, 8]), torch.zeros(2, dtype=D64)
    x = torch.relu(tok)
    assert torch.allclose(OD.camera_head(p, tok), x[:, :9], atol=1e-12)
    p[c + ".fc_fov.0.weight"] = rows([7, 8], -1.0)
    assert torch.allclose(OD.camera_head(p, tok), torch.cat([x[:, :7], torch.zeros(3, 2, dtype=D64)], 1), atol=1e-12)


def test_pose_head_residual_blocks_pool_and_normalisation():
    """mapanything-rs/src/heads.rs:80-99: proj (keeps the d channels, zero-padded to pd), two
    residual blocks x + relu(c3(relu(c2(relu(c1 x))))) with zero weights and biases c_b (so
    x + relu(c_b)), mean pool over the pixels, two relu(Linear = I), q = fc_rot / |fc_rot|
    with fc_rot keeping channels 0-3, t = fc_t keeping 4-6."""
    g = torch.Generator().manual_seed(11)
    V, d, pd, h, w = 2, 6, 10, 3, 4
    feats = rng_t(g, V, d, h, w)
    c = [rng_t(g, pd), rng_t(g, pd)]
    p = {"pose_head.proj.weight": conv1x1(pd, d), "pose_head.proj.bias": torch.zeros(pd, dtype=D64)}
    for b in range(2):
        for k in (1, 2, 3):
            n = f"pose_head.res_conv.{b}.res_conv{k}"
            p[n + ".weight"] = torch.zeros(pd, pd, 1, 1, dtype=D64)
            p[n + ".bias"] = c[b] if k == 3 else torch.zeros(pd, dtype=D64)
    for n in ("more_mlps.0", "more_mlps.2"):
        p[f"pose_head.{n}.weight"], p[f"pose_head.{n}.bias"] = torch.eye(pd, dtype=D64), torch.zeros(pd, dtype=D64)
    p["pose_head.fc_rot.weight"], p["pose_head.fc_rot.bias"] = torch.eye(pd, dtype=D64)[:4], torch.zeros(4, dtype=D64)
    p["pose_head.fc_t.weight"], p["pose_head.fc_t.bias"] = torch.eye(pd, dtype=D64)[4:7], torch.zeros(3, dtype=D64)
    t, q = OM.pose_head(p, feats)
    x = _embed(feats, pd) + (torch.relu(c[0]) + torch.relu(c[1]))[None, :, None, None]
    pooled = torch.relu(x.mean((2, 3)))
    assert torch.allclose(q, pooled[:, :4] / pooled[:, :4].norm(dim=1, keepdim=True), atol=1e-12)
    assert torch.allclose(t, pooled[:, 4:7], atol=1e-12)


def test_scale_head_has_no_activation_after_the_projection_and_clamps():
    """mapanything-rs/src/heads.rs:122-129: proj (no activation) -> relu(Linear) x2 -> Linear ->
    exp -> clamp >= 1e-8. proj = -I, mlp.0 = -I, mlp.1 = I, output = ones: exp(sum relu(tok)),
    where a ReLU after the projection would give exp(0). A very negative output clamps."""
    n = 5
    g = torch.Generator().manual_seed(12)
    tok = rng_t(g, 1, n)
    z = torch.zeros(n, dtype=D64)
    p = {"scale_head.proj.weight": -torch.eye(n, dtype=D64), "scale_head.proj.bias": z,
         "scale_head.mlp.0.0.weight": -torch.eye(n, dtype=D64), "scale_head.mlp.0.0.bias": z,
         "scale_head.mlp.1.0.weight": torch.eye(n, dtype=D64), "scale_head.mlp.1.0.bias": z,
         "scale_head.output_proj.weight": torch.ones(1, n, dtype=D64),
         "scale_head.output_proj.bias": torch.zeros(1, dtype=D64)}
    assert torch.allclose(OM.scale_head(p, tok), torch.exp(torch.relu(tok).sum()).reshape(1), atol=1e-12)
    assert float(torch.relu(tok).sum()) > 0.1
    p["scale_head.output_proj.weight"] = torch.zeros(1, n, dtype=D64)
    p["scale_head.output_proj.bias"] = torch.full((1,), -200.0, dtype=D64)
    assert float(OM.scale_head(p, tok)) == 1e-8


def test_dense_output_rays_depth_conf_and_mask():
    """mapanything-rs/src/model.rs:148-172: |point| = exp(raw3) * scale along raw[0:3]'s
    direction, a zero ray (norm clamped at 1e-8) gives the zero point, conf = 1 + exp(raw4),
    mask = raw5 > 0."""
    g = torch.Generator().manual_seed(13)
    raw = rng_t(g, 2, 6, 3, 4)
    raw[0, 0:3, 0, 0] = 0.0
    scale = 2.5
    pts, conf, mask = OM.dense_output(raw, scale)
    n = pts.norm(dim=1)
    want_n = torch.exp(raw[:, 3]) * scale
    want_n[0, 0, 0] = 0.0
    assert torch.allclose(n, want_n, atol=1e-12)
    cosang = (pts * raw[:, 0:3]).sum(1) / (n * raw[:, 0:3].norm(dim=1) + 1e-300)
    cosang[0, 0, 0] = 1.0
    assert torch.allclose(cosang, torch.ones_like(cosang), atol=1e-12)
    assert torch.equal(conf, 1 + torch.exp(raw[:, 4])) and torch.equal(mask, raw[:, 5] > 0)


# --- info sharing: mapanything-rs/src/info_sharing.rs:50-102 ---------------------------------

def _info_params(spec, g, mode):
    """mode "const": block i adds c_i to the tokens it runs over (attention branch = proj bias,
    LayerScale 1 / 0); mode "mean": uniform attention of v = LN1(x) (q = k = 0, v and proj
    identities), so a block adds the mean of LN1(x) over the tokens it attends within."""
    d = spec.info_dim
    p = {}
    cs = []
    for i in range(spec.info_depth):
        n = f"info_sharing.self_attention_blocks.{i}"
        bp, _ = _block_params(g, d, spec.info_hidden, n)
        p.update(bp)
        p[n + ".norm1.weight"], p[n + ".norm1.bias"] = torch.ones(d, dtype=D64), torch.zeros(d, dtype=D64)
        p[n + ".ls1.gamma"], p[n + ".ls2.gamma"] = torch.ones(d, dtype=D64), torch.zeros(d, dtype=D64)
        if mode == "const":
            p[n + ".attn.proj.weight"] = torch.zeros(d, d, dtype=D64)
            cs.append(rng_t(g, d))
            p[n + ".attn.proj.bias"] = cs[-1]
        else:
            p[n + ".attn.qkv.weight"][2 * d:] = torch.eye(d, dtype=D64)
            p[n + ".attn.proj.weight"], p[n + ".attn.proj.bias"] = torch.eye(d, dtype=D64), torch.zeros(d, dtype=D64)
    p["info_sharing.norm.weight"] = 1 + rng_t(g, d, scale=0.1)
    p["info_sharing.norm.bias"] = rng_t(g, d, scale=0.1)
    p["info_sharing.view_pos_table"] = rng_t(g, 1, d)
    p["scale_token"] = rng_t(g, d)
    return p, cs


def _info_inputs(spec, g, V=3, P=4):
    return rng_t(g, V, P, spec.info_dim), rng_t(g, V, 1, spec.info_dim)


def test_info_sharing_hooks_and_which_blocks_see_the_scale_token():
    """Blocks that add a constant c_i: the view tokens after block i hold x + sum_{j<=i} c_j,
    the scale token only the even (global) blocks' c_j (odd blocks run per view while it
    waits). Hooks after blocks 1, 2, 3 (the tiny spec) are LN(.) of those sums; the sequence
    per view is [patches, class] with the view position table on view 0 only."""
    spec = specs.MA_SPECS["tiny"]
    g = torch.Generator().manual_seed(14)
    p, cs = _info_params(spec, g, "const")
    patches, classes = _info_inputs(spec, g)
    per_view, scale_tok = OM.info_sharing_forward(p, spec, patches, classes)
    nw, nb = p["info_sharing.norm.weight"], p["info_sharing.norm.bias"]
    for k, hook in enumerate(spec.hooks):
        add = sum(cs[: hook + 1])
        for v in range(3):
            x = patches[v] + (p["info_sharing.view_pos_table"][0] if v == 0 else 0) + add
            assert torch.allclose(per_view[v][k], ln(x, 1e-6) * nw + nb, atol=1e-12), (k, v)
    s = p["scale_token"] + sum(cs[j] for j in range(spec.hooks[2] + 1) if j % 2 == 0)
    assert torch.allclose(scale_tok, ln(s, 1e-6) * nw + nb, atol=1e-12)


def test_info_sharing_even_blocks_attend_globally_odd_blocks_per_view():
    """Blocks that add the mean of LN1(x) over what they attend within: the even blocks over all
    V*n + 1 tokens (scale token included), the odd blocks over each view's n tokens (the scale
    token unchanged). Computed block by block and compared with the last hook."""
    spec = specs.MA_SPECS["tiny"]
    g = torch.Generator().manual_seed(15)
    p, _ = _info_params(spec, g, "mean")
    patches, classes = _info_inputs(spec, g)
    V, P, d = patches.shape
    n = P + 1
    seq = torch.cat([patches, classes], 1)
    seq[0] = seq[0] + p["info_sharing.view_pos_table"][0]
    x = torch.cat([seq.reshape(V * n, d), p["scale_token"][None]], 0)
    for i in range(spec.info_depth):
        h = ln(x, 1e-6)
        if i % 2 == 0:
            x = x + h.mean(0, keepdim=True)
        else:
            views = x[: V * n].reshape(V, n, d) + h[: V * n].reshape(V, n, d).mean(1, keepdim=True)
            x = torch.cat([views.reshape(V * n, d), x[V * n:]], 0)
    per_view, scale_tok = OM.info_sharing_forward(p, spec, patches, classes)
    nw, nb = p["info_sharing.norm.weight"], p["info_sharing.norm.bias"]
    last = ln(x, 1e-6) * nw + nb
    for v in range(V):
        assert torch.allclose(per_view[v][2], last[v * n: v * n + P], atol=1e-12)
    assert torch.allclose(scale_tok, last[V * n], atol=1e-12)


def test_mapanything_patches_are_fusion_normed_and_the_class_token_is_raw():
    """mapanything-rs/src/model.rs:104-110: the info transformer gets LN_fusion(patches) and the
    raw class token. With info blocks that add the per-view mean of LN1(x) (odd blocks) or
    the global mean (even blocks) the class token reaches every patch, so forward()'s info
    stream after the last block must equal info_sharing_forward fed (fused patches, raw
    class); feeding a fusion-normed class token instead gives another stream."""
    spec = specs.MA_SPECS["tiny"]
    g = torch.Generator().manual_seed(16)
    w = synth.generate(synth.ma_shapes(spec), seed=16, layer_scale=1.0)
    p = C.to_torch(w, D64)
    ip, _ = _info_params(spec, g, "mean")
    p.update(ip)
    images = torch.from_numpy(synth.uniform_images(2, 28, 42, seed=3)).to(D64)
    enc_taps, info_taps = [], []
    OM.forward(p, spec, images, dtype=D64, taps=enc_taps, info_taps=info_taps)
    tokens = enc_taps[-1]
    fused = ln(tokens[:, 1:], 1e-6) * p["fusion_norm_layer.weight"] + p["fusion_norm_layer.bias"]
    raw_cls, normed_cls = tokens[:, :1], ln(tokens[:, :1], 1e-6) * p["fusion_norm_layer.weight"] + p["fusion_norm_layer.bias"]
    want, wrong = [], []
    OM.info_sharing_forward(p, spec, fused, raw_cls, taps=want)
    OM.info_sharing_forward(p, spec, fused, normed_cls, taps=wrong)
    assert len(info_taps) == len(want) == spec.info_depth
    assert torch.allclose(info_taps[-1], want[-1], atol=1e-10)
    assert not torch.allclose(wrong[-1], want[-1], atol=1e-6)


# --- token assembly and forward wiring: mapanything-rs/src/{dinov2.rs:129-145, model.rs:86-144},
# depthanything3-rs/src/backbone.rs:140-163 ---------------------------------------------------

def patch_embed(images, w, b):
    """Conv2d(3, d, 14, stride 14) from its definition: each 14x14 patch flattened in (channel,
    row, column) order against the [d, 3, 14, 14] kernel, plus the bias."""
    V, ch, H, W = images.shape
    R, Cc = H // 14, W // 14
    cols = images.reshape(V, ch, R, 14, Cc, 14).permute(0, 2, 4, 1, 3, 5).reshape(V, R * Cc, ch * 196)
    return cols @ w.reshape(w.shape[0], -1).T + b


def _embedded_tokens(p, prefix, images):
    """cat(cls, patch_embed(x)) + pos over all 1 + P slots (class slot = cls + pos_embed[0, 0])."""
    V, _, H, W = images.shape
    R, Cc = H // 14, W // 14
    pos = C.positional_embedding(p[prefix + ".pos_embed"], R, Cc)[0].to(D64)
    assert torch.equal(pos[0], p[prefix + ".pos_embed"][0, 0].float().to(D64))  # class slot not resized
    pe = patch_embed(images, p[prefix + ".patch_embed.proj.weight"], p[prefix + ".patch_embed.proj.bias"])
    cls = p[prefix + ".cls_token"].reshape(1, 1, -1).expand(V, 1, pe.shape[-1])
    return torch.cat([cls, pe], 1) + pos


def test_mapanything_encoder_token_assembly_closed_form():
    """mapanything-rs/src/dinov2.rs:129-145 with LayerScale 0 (every block the identity): the
    encoder returns cat(cls, patch_embed(x)) + pos over all 1 + P slots. Fails if the class token
    is appended last, if the positional embedding skips the class slot, or if a final norm is
    applied (the reference's encoder has none)."""
    spec = specs.MA_SPECS["tiny"]
    w = synth.generate(synth.ma_shapes(spec), seed=21, layer_scale=0.0)
    p = C.to_torch(w, D64)
    p["encoder.model.cls_token"] = p["encoder.model.cls_token"] * 50      # well away from pos and the patches
    images = torch.from_numpy(synth.uniform_images(2, 28, 42, seed=4)).to(D64)
    got = OM.encoder_forward(p, spec, images)
    want = _embedded_tokens(p, "encoder.model", images)
    assert got.shape == (2, 7, spec.enc_dim)
    assert torch.allclose(got, want, atol=1e-12)
    # forward() hands the same tokens on (encoder_only): no norm between encoder and caller
    out = OM.forward(p, spec, images, dtype=D64, encoder_only=True)
    assert torch.allclose(out["encoder_tokens"].to(D64), want, atol=1e-5)


def _mean_block_0(p, prefix, d):
    """Block 0 adds each sequence's mean of LN(x) over its tokens (q = k = 0: uniform attention;
    v = LN1(x) with norm1 weight 1 / bias 0; proj I; LayerScale 1, feed-forward LayerScale 0)."""
    n = f"{prefix}.blocks.0"
    p[n + ".norm1.weight"], p[n + ".norm1.bias"] = torch.ones(d, dtype=D64), torch.zeros(d, dtype=D64)
    qkv = torch.zeros(3 * d, d, dtype=D64)
    qkv[2 * d:] = torch.eye(d, dtype=D64)
    p[n + ".attn.qkv.weight"], p[n + ".attn.qkv.bias"] = qkv, torch.zeros(3 * d, dtype=D64)
    p[n + ".attn.proj.weight"], p[n + ".attn.proj.bias"] = torch.eye(d, dtype=D64), torch.zeros(d, dtype=D64)
    p[n + ".ls1.gamma"], p[n + ".ls2.gamma"] = torch.ones(d, dtype=D64), torch.zeros(d, dtype=D64)


def test_da3_class_slot_carries_pos0_into_the_reference_view_choice():
    """depthanything3-rs/src/backbone.rs:140-163: the class slot starts as cls + pos_embed[0, 0]
    (the positional embedding covers all 1 + P slots), and the saddle-balanced selection before
    block alt_start - 1 reads it. Block 0 adds each view's mean of LN(x) over its n tokens and
    every other block is the identity (LayerScale 0), so the selection sees cls + pos[0] +
    mean_t LN(x_t), computed here from first principles; the selection itself is pinned by
    reference_view.rs's KATs (test_oracle.py). The weights are chosen so that dropping pos[0]
    from the class slot selects another view (asserted below), besides changing the tap."""
    spec = specs.DA3_VARIANTS["small"]
    d = spec.dim
    b = "model.backbone.pretrained"
    w = synth.generate(synth.da3_shapes(spec), seed=23, layer_scale=0.0)
    p = C.to_torch(w, D64)
    g = torch.Generator().manual_seed(4)
    pos = p[b + ".pos_embed"].clone()
    pos[0, 0] = rng_t(g, d, scale=1.0)
    p[b + ".pos_embed"] = pos
    _mean_block_0(p, b, d)
    V = 5
    images = torch.from_numpy(synth.procedural_images(V, 28, 42, seed=24)).to(D64)
    taps = []
    layers, cam, ref = OD.backbone_forward(p, spec, images, OD.REF_SADDLE, taps=taps)
    x = _embedded_tokens(p, b, images)
    cls_after = x[:, 0] + ln(x, 1e-6).mean(1)
    assert torch.allclose(taps[0][:, 0], cls_after, atol=1e-12)
    assert torch.allclose(taps[spec.alt_start - 2][:, 0], cls_after, atol=1e-12)
    want = OD.select_reference_view(cls_after.float().numpy(), OD.REF_SADDLE)
    assert ref == want == 3
    # the test discriminates: without pos[0] on the class slot the choice moves
    x_slip = x.clone()
    x_slip[:, 0] -= pos[0, 0].float().to(D64)
    slip = OD.select_reference_view((x_slip[:, 0] + ln(x_slip, 1e-6).mean(1)).float().numpy(), OD.REF_SADDLE)
    assert slip != want, (slip, want)


def test_mapanything_forward_wiring():
    """mapanything-rs/src/model.rs:86-144 with a closed-form encoder (LayerScale 0) and info blocks
    that each add a constant c_i (proj bias, LayerScale 1 / 0): the dense head's hooks are
    [LN_fusion(patches), LN(x + sum c) after each hook block], hook 0 being the fusion-normed
    encoder patches (model.rs:106, not the raw tokens); the pose head reads the normed last hook
    (model.rs:132); the scale head reads the normed scale token of the last hook; translation is
    fc_t times the scale (model.rs:140). The DPT, pose and scale heads are pinned by their own
    closed forms above and are called here on inputs computed from first principles."""
    spec = specs.MA_SPECS["tiny"]
    g = torch.Generator().manual_seed(25)
    w = synth.generate(synth.ma_shapes(spec), seed=25, layer_scale=0.0)
    p = C.to_torch(w, D64)
    ip, cs = _info_params(spec, g, "const")
    p.update(ip)
    p["scale_head.output_proj.bias"] = p["scale_head.output_proj.bias"] + 0.7    # scale well away from 1
    V, R, Cc = 3, 2, 3
    images = torch.from_numpy(synth.procedural_images(V, 28, 42, seed=26)).to(D64)
    out = OM.forward(p, spec, images, dtype=D64)

    tokens = _embedded_tokens(p, "encoder.model", images)
    fused = ln(tokens[:, 1:], 1e-6) * p["fusion_norm_layer.weight"] + p["fusion_norm_layer.bias"]
    nw, nb = p["info_sharing.norm.weight"], p["info_sharing.norm.bias"]
    vp = p["info_sharing.view_pos_table"][0]
    hooks = [fused]
    for hk in spec.hooks:
        x = fused + sum(cs[: hk + 1])
        x[0] = x[0] + vp
        hooks.append(ln(x, 1e-6) * nw + nb)
    s = p["scale_token"] + sum(cs[j] for j in range(spec.hooks[2] + 1) if j % 2 == 0)
    scale = OM.scale_head(p, (ln(s, 1e-6) * nw + nb)[None])[0]
    raw = OM.dpt_forward(p, spec, hooks, R, Cc)
    spatial = hooks[3].transpose(1, 2).reshape(V, spec.info_dim, R, Cc)
    trans, quat = OM.pose_head(p, spatial)
    assert abs(float(scale) - 1.0) > 0.3
    assert abs(out["scale"] - float(scale)) < 1e-12
    assert torch.allclose(out["raw"].to(D64), raw, atol=1e-10)
    assert torch.allclose(out["quaternion"].to(D64), quat, atol=1e-6)
    assert torch.allclose(out["translation_raw"].to(D64), trans, atol=1e-6)
    assert torch.allclose(out["translation"].to(D64), trans * scale, atol=1e-6)
    pts, conf, mask = OM.dense_output(raw, scale)
    assert torch.allclose(out["points"].to(D64), pts, atol=1e-5)
    assert torch.equal(out["mask"], mask)
