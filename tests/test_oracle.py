"""CPU checks that pin the oracle (oracle/) before it is trusted as the parity reference.

Each restated function is pinned by at least one of:
  * the known-answer tests of the reference's own unit tests, restated (file:line cited);
  * a library routine with the same semantics (PyTorch CPU);
  * a closed form / invariant / brute force chosen so a plausible slip (sign, index, order of
    concatenation, swapped axis) fails.
The composite network order has no reference golden vector (the reference never checks its
network numerically); it is pinned by the per-function checks here, the structural
closed forms below (LayerScale 0, view permutation) and the committed golden fixtures.
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


# --- RoPE: depthanything3-rs/src/rope.rs:79-106, backbone.rs:203-212 -------------------

def test_rope_position_zero_is_identity():
    cos, sin = C.rope_tables([(0, 0)])
    x = torch.arange(64, dtype=torch.float32).reshape(1, 1, 1, 64)
    assert torch.max(torch.abs(C.rope_apply(x, cos, sin) - x)) < 1e-6


def test_rope_rotation_keeps_the_norm_and_follows_the_row():
    cos, sin = C.rope_tables([(3, 0)])
    x = torch.zeros(1, 1, 1, 64)
    x[..., 0] = 1.0
    x[..., 32] = 2.0
    out = C.rope_apply(x, cos, sin).flatten()
    assert abs(out[0] - math.cos(3.0)) < 1e-6
    assert abs(out[16] - math.sin(3.0)) < 1e-6
    assert abs(out[32] - 2.0) < 1e-6
    assert abs(out.norm() - math.sqrt(5.0)) < 1e-5


def test_rope_column_axis_and_frequency():
    # column 5 rotates the second half; pair p uses frequency 100^(-p/16)
    cos, sin = C.rope_tables([(0, 5)])
    x = torch.zeros(1, 64)
    x[0, 32 + 3] = 1.0
    out = C.rope_apply(x, cos, sin).flatten()
    ang = 5.0 / 100.0 ** (3 / 16)
    assert abs(out[32 + 3] - math.cos(ang)) < 1e-6
    assert abs(out[32 + 16 + 3] - math.sin(ang)) < 1e-6
    assert torch.count_nonzero(out[:32]) == 0


def test_rope_positions_follow_the_grid():
    within = OD.rope_positions(2, 3, False)
    assert within[0] == (0, 0) and within[1] == (1, 1) and within[3] == (1, 3) and within[4] == (2, 1)
    assert all(p == (1, 1) for p in OD.rope_positions(2, 3, True)[1:])


# --- uv embedding: depthanything3-rs/src/uv_embed.rs:58-74 --------------------------------

def test_uv_corners_sit_at_the_shrunk_span():
    emb = OD.uv_embedding(8, 2, 4, 2.0).flatten().numpy()
    u = -2.0 / math.sqrt(5.0) * 0.75
    assert abs(emb[0] - math.sin(u) * 0.1) < 1e-6
    v = 1.0 / math.sqrt(5.0) * 0.5
    assert abs(emb[4 * 8 + 4] - math.sin(v) * 0.1) < 1e-6


def test_uv_embedding_is_symmetric_and_bounded():
    emb = OD.uv_embedding(16, 5, 7, 7 / 5)[0].numpy()
    # sin(u) is odd in the column, cos(u) even; |values| <= 0.1
    assert np.allclose(emb[0:4, :, ::-1], -emb[0:4], atol=1e-7)
    assert np.allclose(emb[4:8, :, ::-1], emb[4:8], atol=1e-7)
    assert np.allclose(emb[8:12, ::-1, :], -emb[8:12], atol=1e-7)
    assert np.max(np.abs(emb)) <= 0.1 + 1e-7


# --- bicubic resize: mapanything-rs/src/dinov2.rs:152-165 + torch library routine ----------

def test_bicubic_weights_sum_to_one():
    for t in (0.0, 0.25, 0.5, 0.9):
        assert abs(sum(C.bicubic_weights(t)) - 1.0) < 1e-12
    assert C.bicubic_weights(0.0) == [0.0, 1.0, 0.0, 0.0]


def test_resize_to_same_size_with_unit_scale_is_identity():
    grid = np.arange(2 * 3 * 2, dtype=np.float32)
    assert np.array_equal(C.resize_grid(grid, 2, 3, 2, 3, 1.0, 1.0).ravel(), grid)


@pytest.mark.parametrize("rows,cols", [(27, 36), (28, 37), (36, 36), (4, 3)])
def test_resize_grid_matches_torch_bicubic(rows, cols):
    """The DINOv2 resize is F.interpolate(bicubic, align_corners=False, scale_factor) with
    scale (out + 0.1) / 37, which the reference restates by hand (dinov2.rs:20-76)."""
    g = np.random.default_rng(0).standard_normal((37, 37, 5)).astype(np.float32)
    ours = C.resize_grid(g, 37, 37, rows, cols, (rows + 0.1) / 37, (cols + 0.1) / 37)
    x = torch.from_numpy(g).double().permute(2, 0, 1)[None]
    ref = F.interpolate(x, scale_factor=((rows + 0.1) / 37, (cols + 0.1) / 37), mode="bicubic",
                        align_corners=False, recompute_scale_factor=False)[0].permute(1, 2, 0).numpy()
    assert ref.shape == ours.shape
    assert np.max(np.abs(ours - ref)) < 1e-5


# --- reference view: depthanything3-rs/src/reference_view.rs:104-123 ----------------------

def test_reorders_and_restores():
    order = OD.order_with_reference_first(5, 2)
    assert order == [2, 0, 1, 3, 4]
    assert OD.positions_of_views(order) == [1, 2, 0, 3, 4]


def test_fewer_than_three_views_keep_the_first():
    assert OD.select_reference_view(np.array([[1.0, 0.0], [0.0, 1.0]]), OD.REF_MIDDLE) == 0


def test_saddle_balanced_picks_the_median_view():
    tokens = np.array([[1.0, 0.0, 0.0, 0.1], [1.0, 0.5, 0.0, 0.2], [1.0, 1.0, 0.0, 0.3]])
    assert OD.select_reference_view(tokens, OD.REF_SADDLE) == 1


def test_saddle_balanced_is_permutation_equivariant():
    rng = np.random.default_rng(3)
    tokens = rng.standard_normal((6, 32))
    best = OD.select_reference_view(tokens, OD.REF_SADDLE)
    perm = rng.permutation(6)
    assert perm[OD.select_reference_view(tokens[perm], OD.REF_SADDLE)] == best


# --- camera: depthanything3-rs/src/camera_head.rs:97-115 -----------------------------------

def test_identity_encoding_is_the_identity_pose():
    R = OD.quaternion_to_rotation(0.0, 0.0, 0.0, 1.0)
    assert np.linalg.norm(R - np.eye(3)) < 1e-12
    fx, _ = OD.focal(1.0, 1.0, 100, 200)
    assert abs(fx - 100.0 / math.tan(0.5)) < 1e-9


def test_non_unit_quaternion_rotates_like_its_direction():
    s = 2.0 * math.sin(math.pi / 4)
    R = OD.quaternion_to_rotation(0.0, 0.0, s, s)
    assert np.linalg.norm(R @ np.array([1.0, 0.0, 0.0]) - np.array([0.0, 1.0, 0.0])) < 1e-6


# --- variants: depthanything3-rs/src/variant.rs:158-181; vit_block.rs:114-117 ----------------

def test_variant_invariants():
    for name, s in specs.DA3_VARIANTS.items():
        assert s.dim == s.heads * 64, name
        assert s.alt_start < s.out_layers[0], name
        assert all(a < b for a, b in zip(s.out_layers, s.out_layers[1:])), name
        assert s.out_layers[3] == s.depth - 1, name


def test_swiglu_width_matches_dinov2_giant():
    assert specs.swiglu_hidden_dim(1536) == 4096


# --- elementary ops ------------------------------------------------------------------------

def test_blockwise_attention_matches_one_shot_softmax():
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(2, 3, 300, 64, generator=g, dtype=torch.float64) for _ in range(3))
    ref = torch.softmax(q @ k.transpose(-1, -2) / 8.0, -1) @ v
    assert torch.max(torch.abs(C.attention(q, k, v, chunk=64) - ref)) < 1e-12


def test_rotate_pairs_is_a_quarter_turn():
    x = torch.randn(5, 64, dtype=torch.float64)
    r = C.rotate_pairs(x)
    assert torch.allclose(C.rotate_pairs(r), -x)                 # two quarter turns
    assert torch.allclose((x * r).sum(-1), torch.zeros(5, dtype=torch.float64))  # orthogonal


def test_conv_transpose_with_kernel_equal_stride_is_a_pixel_shuffle_gemm():
    """ConvTranspose2d(k = s) semantics (weight [in, out, kh, kw]) by brute force."""
    g = torch.Generator().manual_seed(1)
    x = torch.randn(1, 3, 2, 2, generator=g, dtype=torch.float64)
    w = torch.randn(3, 4, 2, 2, generator=g, dtype=torch.float64)
    out = F.conv_transpose2d(x, w, stride=2)
    brute = torch.zeros(1, 4, 4, 4, dtype=torch.float64)
    for r in range(2):
        for c in range(2):
            for dy in range(2):
                for dx in range(2):
                    brute[0, :, 2 * r + dy, 2 * c + dx] = torch.einsum("i,io->o", x[0, :, r, c], w[:, :, dy, dx])
    assert torch.allclose(out, brute)


def test_bilinear_align_corners_brute_force():
    x = torch.arange(12, dtype=torch.float64).reshape(1, 1, 3, 4)
    out = C.resize_bilinear(x, 5, 7)
    # corners are kept exactly; the centre is the mean of its neighbours by construction
    assert out[0, 0, 0, 0] == 0 and out[0, 0, -1, -1] == 11 and out[0, 0, 0, -1] == 3 and out[0, 0, -1, 0] == 8
    y, xx = 3 * (2 / 4), 6 * (3 / 6)
    y0, x0 = int(y), int(xx)
    ly, lx = y - y0, xx - x0
    a = x[0, 0]
    ref = (1 - ly) * ((1 - lx) * a[y0, x0] + lx * a[y0, min(x0 + 1, 3)]) + ly * ((1 - lx) * a[min(y0 + 1, 2), x0] + lx * a[min(y0 + 1, 2), min(x0 + 1, 3)])
    assert abs(out[0, 0, 3, 6] - ref) < 1e-12


# --- structural closed forms of the composite forward ------------------------------------

def test_da3_layerscale_zero_makes_every_block_the_identity():
    """With both LayerScales 0 each block returns its input, so every hook is
    cat(x, norm(x)) of the embedded tokens (camera token swapped in at alt_start) and the
    camera tokens are cat(camera token, camera token): catches a swapped concat or a norm
    applied to the wrong half."""
    spec = specs.DA3_VARIANTS["small"]
    w = synth.generate(synth.da3_shapes(spec), seed=2, layer_scale=0.0)
    p = C.to_torch(w)
    images = torch.from_numpy(synth.uniform_images(2, 28, 42, seed=1))
    layers, cam, ref = OD.backbone_forward(p, spec, images, OD.REF_FIRST)
    b = "model.backbone.pretrained"
    patches = C.conv(images, p, b + ".patch_embed.proj", stride=14).flatten(2).transpose(1, 2)
    x0 = patches + C.positional_embedding(p[b + ".pos_embed"], 2, 3)[:, 1:]
    normed = C.layer_norm(x0, p[b + ".norm.weight"], p[b + ".norm.bias"], 1e-5)
    for layer in layers:
        assert torch.allclose(layer, torch.cat([x0, normed], -1), atol=1e-6)
    camt = p[b + ".camera_token"][0]
    assert torch.allclose(cam[0], torch.cat([camt[0], camt[0]]))
    assert torch.allclose(cam[1], torch.cat([camt[1], camt[1]]))


def test_mapanything_views_after_the_first_are_equivariant():
    spec = specs.MA_SPECS["tiny"]
    w = synth.generate(synth.ma_shapes(spec), seed=4, layer_scale=1.0)
    images = synth.procedural_images(3, 28, 42, seed=2)
    a = OM.forward(w, spec, images)
    b = OM.forward(w, spec, images[[0, 2, 1]])
    assert torch.allclose(b["raw"], a["raw"][[0, 2, 1]], atol=1e-5)
    assert abs(a["scale"] - b["scale"]) < 1e-5


def test_da3_outputs_are_positive_and_rays_finite():
    spec = specs.DA3_VARIANTS["small"]
    w = synth.generate(synth.da3_shapes(spec), seed=5, layer_scale=1.0)
    out = OD.forward_raw(w, spec, synth.procedural_images(3, 28, 42, seed=3))
    assert torch.all(out["depth"] > 0) and torch.all(out["depth_conf"] > 1)
    assert torch.isfinite(out["ray_logits"]).all() and out["ray_logits"].shape == (3, 7, 16, 24)
    assert out["pose_encoding"].shape == (3, 9) and torch.all(out["pose_encoding"][:, 7:] >= 0)


# --- known-camera ray encoder (mapanything-rs/src/{model.rs:38-54, ray_encoder.rs}) -----------

def test_pixel_unshuffle_orders_channel_then_row_then_column():
    # KAT of mapanything-rs/src/ray_encoder.rs:93-103: one channel, 2x4 image, factor 2
    x = torch.arange(8.0).reshape(1, 1, 2, 4)
    out = OM.pixel_unshuffle(x, 2)[0]
    assert out.tolist() == [[[0.0, 2.0]], [[1.0, 3.0]], [[4.0, 6.0]], [[5.0, 7.0]]]
    # and torch's PixelUnshuffle (the routine the reference names) at the encoder's factor
    y = torch.randn(2, 3, 28, 42)
    assert torch.equal(OM.pixel_unshuffle(y, 14), F.pixel_unshuffle(y, 14))


def test_ray_map_is_a_unit_pinhole_direction():
    fx, fy, cx, cy = 300.0, 250.0, 20.5, 10.0
    r = OM.ray_map((fx, fy, cx, cy), 28, 42).double()
    assert r.shape == (3, 28, 42)
    assert float((r.norm(dim=0) - 1).abs().max()) < 1e-6
    # pixel (x=41, y=0): direction ((41 - cx)/fx, (0 - cy)/fy, 1) normalised
    d = np.array([(41 - cx) / fx, (0 - cy) / fy, 1.0])
    assert np.allclose(r[:, 0, 41].numpy(), d / np.linalg.norm(d), atol=1e-7)
    # the z component is the cosine to the optical axis: largest near the principal point
    assert int(r[2].argmax()) == 10 * 42 + 20


def test_ray_encoder_shortcut_path_closed_form():
    # With conv_in the identity, conv1/conv2 zero and identity shortcuts, each residual block
    # is gelu(0 + x) = gelu(x) (ray_encoder.rs:38-42: the activation follows the add), so the
    # encoder reduces to LN(W @ gelu(gelu(unshuffle(rays)))) with zero-padded channels.
    g = torch.Generator().manual_seed(1)
    e = 64
    w0, w1, w2 = OM.RAY_WIDTHS
    q = "ray_dirs_encoder."
    p = {}
    cin = torch.zeros(w0, w0, 3, 3)
    cin[:, :, 1, 1] = torch.eye(w0)
    p[q + "conv_in.weight"], p[q + "conv_in.bias"] = cin, torch.zeros(w0)
    for i, (a, b) in enumerate(((w0, w1), (w1, w2))):
        k = f"{q}encoder.{i}."
        p[k + "conv1.weight"], p[k + "conv1.bias"] = torch.zeros(b, a, 3, 3), torch.zeros(b)
        p[k + "conv2.weight"], p[k + "conv2.bias"] = torch.zeros(b, b, 3, 3), torch.zeros(b)
        sc = torch.zeros(b, a, 1, 1)
        sc[:a, :, 0, 0] = torch.eye(a)
        p[k + "shortcut.weight"], p[k + "shortcut.bias"] = sc, torch.zeros(b)
    W = torch.randn(e, w2, generator=g) * 0.05
    p[q + "encoder.2.weight"], p[q + "encoder.2.bias"] = W[:, :, None, None], torch.zeros(e)
    lw, lb = 1 + 0.1 * torch.randn(e, generator=g), 0.1 * torch.randn(e, generator=g)
    p[q + "norm_layer.weight"], p[q + "norm_layer.bias"] = lw, lb
    rays = OM.ray_map((60.0, 70.0, 21.0, 13.0), 28, 42)[None]
    got = OM.ray_encoder(p, rays)[0]
    u = OM.pixel_unshuffle(rays, 14)[0].reshape(w0, -1).T          # [P, 588]
    z = torch.zeros(u.shape[0], w2)
    z[:, :w0] = F.gelu(F.gelu(u))
    want = F.layer_norm(z @ W.T, (e,), lw, lb, 1e-6)
    assert torch.allclose(got, want, atol=1e-5)


def test_mapanything_unknown_cameras_match_no_intrinsics():
    spec = specs.MA_SPECS["tiny"]
    w = synth.generate(synth.ma_shapes(spec), seed=3)
    images = synth.procedural_images(2, 28, 42, seed=2)
    a = OM.forward(w, spec, images)
    b = OM.forward(w, spec, images, intrinsics=[None, None])
    c = OM.forward(w, spec, images, intrinsics=[(50.0, 50.0, 21.0, 14.0), None])
    assert torch.equal(a["raw"], b["raw"])
    assert not torch.equal(a["raw"], c["raw"])


# --- post-forward geometry (oracle/geometry.py) ----------------------------------------------

from oracle import geometry as OG


def test_cleaning_zeroes_the_less_confident_point_in_front():
    # KAT of mapanything-rs/src/cleaning.rs:83-103: two cameras at the origin looking down z;
    # image 0 sees a point at depth 1 (conf 2), image 1 one at depth 2 behind it (conf 3).
    points = np.array([[[[0, 0, 1.0]]], [[[0, 0, 2.0]]]], np.float32)
    conf = np.array([[[2.0]], [[3.0]]], np.float32)
    depths = np.array([[[1.0]], [[2.0]]], np.float32)
    cams = [{"R": np.eye(3), "t": np.zeros(3), "focal": 1.0, "pp": np.zeros(2)}] * 2
    out = OG.clean(points, conf, depths, np.ones((2, 1, 1), bool), cams)
    assert out[0, 0, 0] == 0.0 and out[1, 0, 0] == 3.0
    # background points are never zeroed, and equal confidence keeps both
    assert OG.clean(points, conf, depths, np.array([[[False]], [[True]]]), cams)[0, 0, 0] == 2.0
    assert OG.clean(points, np.full_like(conf, 3.0), depths, np.ones((2, 1, 1), bool), cams)[0, 0, 0] == 3.0


def test_relative_to_first_is_identity_for_the_first_view():
    rng = np.random.default_rng(0)
    poses = []
    for _ in range(3):
        q = rng.normal(size=4)
        poses.append((OD.quaternion_to_rotation(*q), rng.normal(size=3)))
    rel = OG.relative_to_first(poses)
    assert np.allclose(rel[0][0], np.eye(3)) and np.allclose(rel[0][1], 0)
    R0, t0 = poses[0]
    for (R, t), (Rr, tr) in zip(poses, rel):           # composing with the first pose undoes it
        assert np.allclose(R0 @ Rr, R) and np.allclose(R0 @ tr + t0, t)


def test_fit_intrinsics_recovers_a_pinhole_camera():
    rng = np.random.default_rng(1)
    H, W, fx, fy, cx, cy = 60, 110, 91.5, 88.0, 52.25, 31.5
    xs, ys = np.meshgrid(np.arange(W, dtype=np.float64), np.arange(H, dtype=np.float64))
    z = rng.uniform(0.5, 4.0, size=(H, W))
    pts = np.stack([(xs - cx) / fx * z, (ys - cy) / fy * z, z], -1).astype(np.float32)
    centre, focal = OG.fit_intrinsics(pts)
    assert np.allclose(centre, [cx, cy], atol=1e-3) and np.allclose(focal, [fx, fy], rtol=1e-5)


def test_unprojection_projects_back_to_its_pixel():
    rng = np.random.default_rng(2)
    depth = rng.uniform(0.5, 3.0, size=(7, 9))
    f, pp = np.array([5.0, 6.0]), np.array([4.5, 3.5])
    p = OG.unproject(depth, f, pp)
    u = f[0] * p[..., 0] / p[..., 2] + pp[0]
    v = f[1] * p[..., 1] / p[..., 2] + pp[1]
    xs, ys = np.meshgrid(np.arange(9), np.arange(7))
    assert np.allclose(u, xs) and np.allclose(v, ys) and np.allclose(p[..., 2], depth)


def test_f64_round_goes_away_from_zero():
    assert OG._round(np.array([2.5, -2.5, 0.4, -0.4, 1.5]).astype(np.float64)).tolist() == [3.0, -3.0, 0.0, -0.0, 2.0]


def test_to_model_input_normalises_and_thresholds_alpha():
    rgba = np.zeros((1, 2, 3, 4), np.uint8)
    rgba[0, 0, 0] = [255, 255, 255, 128]
    rgba[0, 0, 1] = [0, 0, 0, 127]
    rgba[0, 1, 2] = [128, 64, 32, 255]
    img, fg = C.to_model_input(rgba)
    mean, std = np.array(specs.IMAGENET_MEAN), np.array(specs.IMAGENET_STD)
    assert img.shape == (1, 3, 2, 3) and img.dtype == np.float32
    assert np.allclose(img[0, :, 0, 0], (1 - mean) / std, atol=1e-6)
    assert np.allclose(img[0, :, 0, 1], -mean / std, atol=1e-6)
    assert np.allclose(img[0, :, 1, 2], (np.array([128, 64, 32]) / 255 - mean) / std, atol=1e-6)
    assert fg.tolist() == [[[True, False, False], [False, False, True]]]
    # the inverse of the normalisation used by the synthetic images returns the 8-bit values
    back = (img * std[None, :, None, None] + mean[None, :, None, None]) * 255
    assert np.allclose(back, rgba[..., :3].transpose(0, 3, 1, 2), atol=1e-3)
