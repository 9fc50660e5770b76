"""Post-forward reconstruction on the device (splat_da3_reconstruct, splat_ma_reconstruct) against
the oracle's geometry (oracle/geometry.py) applied to the same forward's outputs, so the check
isolates the geometry: cameras from the pose encoding or the intrinsics fit, poses relative to
view 0, unprojection, and the multi-view cleaning.

Tolerances: cameras and fitted intrinsics to 1e-9 of each field's scale (both f64); points are f64 results
stored as f32 (1e-6 relative to the scene extent); confidences after cleaning equal except
where a projection lands within float rounding of a pixel boundary (<= 0.1% of pixels).
"""
import os

import numpy as np
import pytest

from conftest import report

pytestmark = pytest.mark.gpu

from splathip import specs, synth
from oracle import geometry as OG


@pytest.fixture(scope="module")
def da3_path(weights_dir):
    spec = specs.DA3_VARIANTS["small"]
    w = synth.generate(synth.da3_shapes(spec), seed=31, layer_scale=1.0)
    path = os.path.join(str(weights_dir), "geo_da3_small.safetensors")
    synth.save(path, w)
    return path


@pytest.fixture(scope="module")
def ma_path(weights_dir):
    spec = specs.MA_SPECS["tiny"]
    w = synth.generate(synth.ma_shapes(spec), seed=32, layer_scale=1.0)
    path = os.path.join(str(weights_dir), "geo_ma_tiny.safetensors")
    synth.save(path, w)
    return path, spec


def _foreground(V, H, W, seed):
    rng = np.random.default_rng(seed)
    fg = np.ones((V, H, W), np.uint8)
    fg[:, : H // 5] = 0                                 # a background band, as an alpha mask gives
    fg[rng.random((V, H, W)) < 0.05] = 0
    return fg


def _compare(got, ref, tag):
    scene = float(np.abs(ref["points"]).max())
    perr = float(np.abs(got["points"] - ref["points"]).max()) / scene
    cam_err = max(float(np.abs(got[k] - ref[k]).max() / (np.abs(ref[k]).max() + 1e-300))
                  for k in ("rotation", "translation", "focal", "principal_point"))
    diff = float(np.mean(got["conf"] != ref["conf"]))
    zeroed = float(np.mean(ref["conf"] == 0))
    report(tag, points_err=f"{perr:.1e}", cam_err=f"{cam_err:.1e}", conf_mismatch=f"{diff:.1e}", zeroed=f"{zeroed:.3f}")
    assert perr < 1e-6
    assert cam_err < 1e-9
    assert diff <= 1e-3


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("with_fg", [False, True])
def test_da3_reconstruct_matches_the_oracle_geometry(ctx, da3_path, dtype, with_fg):
    images = synth.procedural_images(4, 56, 70, seed=13)
    fg = _foreground(4, 56, 70, seed=1) if with_fg else None
    ctx.load_da3(da3_path, "small", dtype, specs.REF_SADDLE)
    raw = ctx.da3_forward_raw(images)
    got = ctx.da3_reconstruct(images, foreground=fg)
    assert got["reference_view"] == raw["reference_view"]
    assert np.array_equal(got["depth"], raw["depth"])
    ref = OG.da3_reconstruct(raw["depth"], raw["depth_conf"], raw["pose_encoding"], fg)
    _compare(got, ref, f"geometry.da3.{dtype}.fg{int(with_fg)}")
    assert np.allclose(got["rotation"][0], np.eye(3), atol=1e-12) and np.allclose(got["translation"][0], 0, atol=1e-12)


@pytest.mark.parametrize("with_fg", [False, True])
def test_ma_reconstruct_matches_the_oracle_geometry(ctx, ma_path, with_fg):
    path, spec = ma_path
    images = synth.procedural_images(3, 56, 84, seed=14)
    fg = _foreground(3, 56, 84, seed=2) if with_fg else None
    ctx.load_mapanything(path, spec, "f32")
    fwd = ctx.ma_forward(images)
    got = ctx.ma_reconstruct(images, foreground=fg)
    ref = OG.ma_reconstruct(fwd["points"], fwd["conf"], fwd["mask"], fwd["quaternion"], fwd["translation"], fg)
    _compare(got, ref, f"geometry.ma.fg{int(with_fg)}")
    assert np.array_equal(got["depth"], fwd["points"][..., 2])


def test_ma_reconstruct_with_known_cameras(ctx, ma_path):
    path, spec = ma_path
    images = synth.procedural_images(2, 42, 56, seed=15)
    intr = [(40.0, 41.0, 28.0, 21.0), None]
    ctx.load_mapanything(path, spec, "f32")
    fwd = ctx.ma_forward(images, intrinsics=intr)
    got = ctx.ma_reconstruct(images, intrinsics=intr)
    ref = OG.ma_reconstruct(fwd["points"], fwd["conf"], fwd["mask"], fwd["quaternion"], fwd["translation"])
    _compare(got, ref, "geometry.ma.cams")


# --- the geometry alone on crafted outputs (splat_kernel_reconstruct): overlapping views whose
# depths disagree by a few percent, so the cleaning zeroes a large share of the points.

def _small_rotations(rng, V, scale):
    q = np.zeros((V, 4))
    q[:, 3] = 1.0
    q[1:, :3] = rng.normal(scale=scale, size=(V - 1, 3))
    return q / np.linalg.norm(q, axis=1, keepdims=True)


def _run_kernel(ctx, V, H, W, **arrays):
    import torch
    dev = {k: torch.from_numpy(np.ascontiguousarray(v)).cuda() for k, v in arrays.items() if v is not None}
    cams = torch.empty(V, 16, dtype=torch.float64, device="cuda")
    pts = torch.empty(V, H, W, 3, device="cuda")
    conf = torch.empty(V, H, W, device="cuda")
    torch.cuda.synchronize()
    ctx.kernel_reconstruct(V, H, W, **{k: t.data_ptr() for k, t in dev.items()}, cameras=cams.data_ptr(),
                           points=pts.data_ptr(), conf_out=conf.data_ptr())
    ctx.synchronize()
    c = cams.cpu().numpy()
    return {"points": pts.cpu().numpy(), "conf": conf.cpu().numpy(), "rotation": c[:, :9].reshape(V, 3, 3),
            "translation": c[:, 9:12], "focal": c[:, 12:14], "principal_point": c[:, 14:16]}


def test_geometry_kernel_da3_cleaning(ctx):
    rng = np.random.default_rng(5)
    V, H, W = 4, 40, 60
    q = _small_rotations(rng, V, 0.01)
    pose = np.zeros((V, 9), np.float32)
    pose[:, 0:3] = np.concatenate([np.zeros((1, 3)), rng.normal(scale=0.02, size=(V - 1, 3))])
    pose[:, 3:7] = q
    pose[:, 7:9] = [0.9, 1.2]                                  # fov_h, fov_w (radians)
    ys, xs = np.meshgrid(np.arange(H), np.arange(W), indexing="ij")
    base = 2.0 + 0.2 * np.sin(xs / 9.0) * np.cos(ys / 7.0)
    depth = (base[None] * (1 + rng.uniform(-0.06, 0.06, size=(V, H, W)))).astype(np.float32)
    conf = rng.uniform(1.0, 3.0, size=(V, H, W)).astype(np.float32)
    fg = (rng.random((V, H, W)) > 0.1).astype(np.uint8)
    got = _run_kernel(ctx, V, H, W, depth=depth, pose_encoding=pose, conf=conf, foreground=fg)
    ref = OG.da3_reconstruct(depth, conf, pose, fg)
    _compare(got, ref, "geometry.kernel.da3")
    zeroed = float(np.mean(ref["conf"] == 0))
    assert 0.1 < zeroed < 0.9, zeroed                          # the cleaning is exercised
    assert np.all(got["conf"][fg == 0] == conf[fg == 0])      # background keeps its confidence


def test_geometry_kernel_ma_cleaning(ctx):
    rng = np.random.default_rng(6)
    V, H, W = 3, 48, 64
    K = np.array([[52.0, 50.0, 31.5, 23.0], [55.0, 54.0, 32.0, 24.5], [50.0, 51.0, 30.0, 22.0]])
    ys, xs = np.meshgrid(np.arange(H, dtype=np.float64), np.arange(W, dtype=np.float64), indexing="ij")
    pic = np.empty((V, H, W, 3), np.float32)
    for v in range(V):
        d = 3.0 + 0.3 * np.cos(xs / 11.0) + rng.uniform(-0.1, 0.1, size=(H, W))
        fx, fy, cx, cy = K[v]
        pic[v] = np.stack([(xs - cx) / fx * d, (ys - cy) / fy * d, d], -1)
    conf = rng.uniform(1.0, 4.0, size=(V, H, W)).astype(np.float32)
    mask = (rng.random((V, H, W)) > 0.15).astype(np.uint8)
    quat = _small_rotations(rng, V, 0.01).astype(np.float32)
    trans = np.concatenate([np.zeros((1, 3)), rng.normal(scale=0.03, size=(V - 1, 3))]).astype(np.float32)
    got = _run_kernel(ctx, V, H, W, points_in_camera=pic, quaternion=quat, translation=trans, conf=conf, mask=mask)
    ref = OG.ma_reconstruct(pic, conf, mask, quat, trans)
    _compare(got, ref, "geometry.kernel.ma")
    # the fit recovers each view's pinhole camera from its points
    assert np.allclose(got["focal"], K[:, :2], rtol=1e-4) and np.allclose(got["principal_point"], K[:, 2:], atol=1e-3)
    zeroed = float(np.mean(ref["conf"] == 0))
    assert np.mean(mask == 0) + 0.05 < zeroed < 0.9, zeroed   # ambiguous pixels plus cleaned ones


def test_to_model_input_on_the_device(ctx):
    import torch
    from oracle import common as OC
    rng = np.random.default_rng(7)
    rgba = rng.integers(0, 256, size=(3, 28, 42, 4), dtype=np.uint8)
    img = torch.empty(3, 3, 28, 42, device="cuda")
    fg = torch.empty(3, 28, 42, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    ctx.to_model_input_device(rgba, img.data_ptr(), fg.data_ptr())
    ctx.synchronize()
    want_img, want_fg = OC.to_model_input(rgba)
    assert np.array_equal(img.cpu().numpy(), want_img)          # same f32 operations, same order
    assert np.array_equal(fg.cpu().numpy().astype(bool), want_fg)
