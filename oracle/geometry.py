"""CPU oracle for the post-forward geometry — TEST INFRASTRUCTURE ONLY (see oracle/common.py).

Restates in numpy float64:
  * relative_to_first          mapanything-rs/src/reconstruction.rs:22-33
  * DA3 cameras + unprojection depthanything3-rs/src/pipeline.rs:44-112 (camera_head.rs:28-53)
  * fit_intrinsics             mapanything-rs/src/pipeline.rs:18-39
  * MapAnything point maps     mapanything-rs/src/pipeline.rs:41-104
  * multi-view cleaning        mapanything-rs/src/cleaning.rs:28-64
Every function takes the network's outputs (numpy arrays), so the GPU geometry can be checked
on the GPU forward's own outputs.
"""
from __future__ import annotations

import numpy as np

from .da3 import focal as da3_focal, quaternion_to_rotation

DEPTH_TOLERANCE = 0.02          # mapanything-rs/src/cleaning.rs:13
INTRINSICS_SAMPLES_PER_SIDE = 50  # mapanything-rs/src/pipeline.rs:16


def _round(a):
    """f64::round: halves away from zero (numpy's round goes to even)."""
    return np.copysign(np.floor(np.abs(a) + 0.5), a)


def relative_to_first(poses):
    """reconstruction.rs:22-33: (R, t) camera-to-world -> relative to the first camera."""
    R0, t0 = poses[0]
    return [(R0.T @ R, R0.T @ (t - t0)) for R, t in poses]


def da3_cameras(pose_encoding: np.ndarray, height: int, width: int):
    """DepthAnything3::forward's per-view camera (model.rs:127-160, camera_head.rs:28-53):
    rotation from the xyzw quaternion, translation, focal from the two FoVs, the image centre
    as principal point."""
    cams = []
    for e in np.asarray(pose_encoding, np.float64):
        tx, ty, tz, qx, qy, qz, qw, fov_h, fov_w = e[:9]
        cams.append({"R": quaternion_to_rotation(qx, qy, qz, qw), "t": np.array([tx, ty, tz]),
                     "focal": np.array(da3_focal(fov_h, fov_w, height, width)),
                     "pp": np.array([width / 2.0, height / 2.0])})
    return cams


def unproject(depth: np.ndarray, focal, pp) -> np.ndarray:
    """pipeline.rs:44-51: pixel (x, y) at depth d -> ((x - cx)/fx d, (y - cy)/fy d, d), [H, W, 3]."""
    H, W = depth.shape
    d = depth.astype(np.float64)
    xs, ys = np.meshgrid(np.arange(W, dtype=np.float64), np.arange(H, dtype=np.float64))
    return np.stack([(xs - pp[0]) / focal[0] * d, (ys - pp[1]) / focal[1] * d, d], axis=-1)


def clean(points, conf, depths, foreground, cams):
    """cleaning.rs:28-64. points [V, H, W, 3] (scene frame, f32 values), conf [V, H, W],
    depths [V, H, W], foreground [V, H, W] bool, cams: per view R, t (camera to scene), focal
    (one value: the mean of fx, fy) and pp. Returns the new confidences (0 where a point lies
    in front of a more confident foreground point of another view)."""
    V, H, W = conf.shape
    out = conf.copy()
    for i in range(V):
        p = points[i].reshape(-1, 3).astype(np.float64)
        fg_i = foreground[i].reshape(-1)
        c_i = conf[i].reshape(-1)
        zero = np.zeros(p.shape[0], bool)
        for j in range(V):
            if j == i:
                continue
            cam = cams[j]
            q = (p - cam["t"]) @ cam["R"]                      # R^T (p - t), row vectors
            z = q[:, 2]
            ok = fg_i & (z > 0)
            with np.errstate(divide="ignore", invalid="ignore"):
                u = _round(cam["focal"] * q[:, 0] / z + cam["pp"][0])
                v = _round(cam["focal"] * q[:, 1] / z + cam["pp"][1])
            ok &= (u >= 0) & (v >= 0) & (u < W) & (v < H)
            op = np.where(ok, v * W + u, 0).astype(np.int64)
            fg_j = foreground[j].reshape(-1)[op]
            d_j = depths[j].reshape(-1)[op].astype(np.float64)
            c_j = conf[j].reshape(-1)[op]
            zero |= ok & fg_j & (z < (1.0 - DEPTH_TOLERANCE) * d_j) & (c_i < c_j)
        out[i].reshape(-1)[zero] = 0.0
    return out


def da3_reconstruct(depth, depth_conf, pose_encoding, foreground=None):
    """depthanything3-rs/src/pipeline.rs:52-133 on forward_raw's outputs."""
    depth = np.asarray(depth, np.float32)
    V, H, W = depth.shape
    fg = np.ones((V, H, W), bool) if foreground is None else np.asarray(foreground, bool)
    cams = da3_cameras(pose_encoding, H, W)
    poses = relative_to_first([(c["R"], c["t"]) for c in cams])
    points = np.empty((V, H, W, 3), np.float32)
    for v in range(V):
        R, t = poses[v]
        pc = unproject(depth[v], cams[v]["focal"], cams[v]["pp"])
        points[v] = (pc @ R.T + t).astype(np.float32)
    clean_cams = [{"R": R, "t": t, "focal": cams[v]["focal"].mean(), "pp": cams[v]["pp"]}
                  for v, (R, t) in enumerate(poses)]
    conf = clean(points, np.asarray(depth_conf, np.float32), depth, fg, clean_cams)
    return {"points": points, "conf": conf, "rotation": np.stack([R for R, _ in poses]),
            "translation": np.stack([t for _, t in poses]),
            "focal": np.stack([c["focal"] for c in cams]), "principal_point": np.stack([c["pp"] for c in cams])}


def fit_intrinsics(points_in_camera: np.ndarray):
    """mapanything-rs/src/pipeline.rs:18-39: per axis, least-squares (centre, focal) of
    pixel = centre + focal * coordinate / z on every (side/50)-th pixel. Returns (centre, focal)."""
    H, W, _ = points_in_camera.shape
    sy, sx = max(H // INTRINSICS_SAMPLES_PER_SIDE, 1), max(W // INTRINSICS_SAMPLES_PER_SIDE, 1)
    p = points_in_camera[::sy, ::sx].astype(np.float64)
    ys, xs = np.meshgrid(np.arange(0, H, sy, dtype=np.float64), np.arange(0, W, sx, dtype=np.float64), indexing="ij")
    centre, focal = [], []
    for pix, coord in ((xs, p[..., 0]), (ys, p[..., 1])):
        r = (coord / p[..., 2]).ravel()
        pix = pix.ravel()
        N = np.array([[r.size, r.sum()], [r.sum(), (r * r).sum()]])
        c, f = np.linalg.solve(N, np.array([pix.sum(), (r * pix).sum()]))
        centre.append(c)
        focal.append(f)
    return np.array(centre), np.array(focal)


def ma_reconstruct(points_in_camera, conf, mask, quaternion, translation, foreground=None):
    """mapanything-rs/src/pipeline.rs:41-104 on MapAnything::forward's outputs (camera-frame
    points [V, H, W, 3], conf, unambiguous mask, xyzw quaternions, metric translations)."""
    pic = np.asarray(points_in_camera, np.float32)
    V, H, W, _ = pic.shape
    fg = np.ones((V, H, W), bool) if foreground is None else np.asarray(foreground, bool)
    q = np.asarray(quaternion, np.float64)
    t = np.asarray(translation, np.float64)
    poses = relative_to_first([(quaternion_to_rotation(*q[v]), t[v]) for v in range(V)])
    fitted = [fit_intrinsics(pic[v]) for v in range(V)]
    points = np.empty((V, H, W, 3), np.float32)
    for v in range(V):
        R, tv = poses[v]
        points[v] = (pic[v].astype(np.float64) @ R.T + tv).astype(np.float32)
    conf0 = np.where(np.asarray(mask, bool), np.asarray(conf, np.float32), np.float32(0))
    clean_cams = [{"R": R, "t": tv, "focal": fitted[v][1].mean(), "pp": fitted[v][0]} for v, (R, tv) in enumerate(poses)]
    out_conf = clean(points, conf0, pic[..., 2], fg, clean_cams)
    return {"points": points, "conf": out_conf, "rotation": np.stack([R for R, _ in poses]),
            "translation": np.stack([tv for _, tv in poses]),
            "focal": np.stack([f for _, f in fitted]), "principal_point": np.stack([c for c, _ in fitted])}
