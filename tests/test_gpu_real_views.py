"""The reference's own example views through the device preprocessing and the BASELINE-L
MapAnything forward, against the CPU oracle.

Data: instantsplat-rs/web/example/input_view{0..5}.png (six 392x518 RGBA photographs of one
scene, portrait) and cameras.json (their intrinsics), copied unchanged into
tests/golden/example_views/. Portrait views give a 37 x 28 patch grid, the transpose of the
benchmark configurations' 28 x 37.

1. splat_ma_model_inputs on the decoded photos against oracle/preprocess.py (the crate's
   cover-and-crop; Lanczos3's sin may move one u8 level in a few pixels, as in
   test_gpu_preprocess.py).
2. The forward at LayerScale 1 in bf16 and f16 on the device-preprocessed views against the fp32
   oracle on the same input: every block's residual cosine and the outputs, at the conftest.H16
   bounds (mask agreement >= 99%).
3. The same views with their intrinsics (the ray-direction encoder, mapanything-rs/src/model.rs:
   97-102) in f16.
The weights are seeded random (BASELINE-L, N(0, 0.02)); the oracle runs in fp32 on the host's
cores (~12 s a forward on 16 threads).
"""
import json
import os

import numpy as np
import pytest

from conftest import report, H16

pytestmark = [pytest.mark.gpu, pytest.mark.slow]

torch = pytest.importorskip("torch")
Image = pytest.importorskip("PIL.Image")

import splathip
from splathip import specs, synth
from oracle import mapanything as O
from oracle import preprocess as P

HERE = os.path.dirname(os.path.abspath(__file__))
VIEWS = os.path.join(HERE, "golden", "example_views")
SPEC = specs.MA_SPECS["baseline_l"]


def _photos():
    return [np.asarray(Image.open(os.path.join(VIEWS, f"input_view{i}.png")).convert("RGBA")) for i in range(6)]


def _intrinsics():
    with open(os.path.join(VIEWS, "cameras.json")) as f:
        cams = json.load(f)
    return [(c["fx"], c["fy"], c["cx"], c["cy"]) for c in sorted(cams, key=lambda c: c["id"])]


@pytest.fixture(scope="module")
def views(ctx):
    """The device model input of the six photos (and the oracle's, compared here)."""
    photos = _photos()
    W, H = splathip.ma_input_size([(p.shape[1], p.shape[0]) for p in photos])
    report("real_views.inputs", H=H, W=W)
    out = torch.empty(6, 3, H, W, device="cuda")
    fg = torch.empty(6, H, W, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    assert ctx.ma_model_inputs_device(photos, out.data_ptr(), fg.data_ptr()) == (H, W)
    ctx.synchronize()
    got, gfg = out.cpu().numpy(), fg.cpu().numpy().astype(bool)
    ref, rfg = P.ma_model_inputs(photos)
    d = np.abs(got - ref)
    report("real_views.inputs.diff", max=f"{d.max():.2e}", frac_diff=f"{(d > 1e-6).mean():.2e}")
    # one level of a u8 channel is 1/255/std <= 0.0175 after normalisation
    assert d.max() <= 0.018 and (d > 1e-6).mean() < 1e-3
    assert np.array_equal(gfg, rfg)
    return got


@pytest.fixture(scope="module")
def weights(weights_dir):
    w = synth.generate(synth.ma_shapes(SPEC), seed=43, layer_scale=1.0)
    path = os.path.join(str(weights_dir), "ma_baseline_l_real_views.safetensors")
    synth.save(path, w)
    return path, w


def tcos(a, b):
    x = torch.as_tensor(np.asarray(a)).reshape(-1).double()
    y = torch.as_tensor(np.asarray(b)).reshape(-1).double()
    return float((x * y).sum() / (x.norm() * y.norm() + 1e-300))


def _oracle(w, images, intrinsics=None):
    enc_taps, info_taps = [], []
    torch.set_num_threads(max(1, min(16, os.cpu_count() or 1)))
    ref = O.forward(w, SPEC, images, intrinsics=intrinsics, taps=enc_taps, info_taps=info_taps)
    return ref, enc_taps + info_taps


def _check(name, ctx, path, dtype, images, ref, rtaps, intrinsics=None):
    cos_min, med_max = H16[dtype]
    ctx.load_mapanything(path, SPEC, dtype)
    res = {}
    ctx.set_debug_taps(lambda b, x: res.__setitem__(b, tcos(x, rtaps[b])))
    try:
        out = ctx.ma_forward(images, intrinsics=intrinsics)
    finally:
        ctx.set_debug_taps(None)
    assert sorted(res) == list(range(SPEC.enc_depth + SPEC.info_depth))
    worst = min(res.items(), key=lambda kv: kv[1])
    depth = np.exp(out["raw"][:, 3].astype(np.float64)) * out["scale"][0]
    rdepth = np.exp(ref["raw"][:, 3].double().numpy()) * ref["scale"]
    med = float(np.median(np.abs(depth / rdepth - 1)))
    cos = {k: tcos(out[k], r) for k, r in (("raw", ref["raw"]), ("points", ref["points"].permute(0, 2, 3, 1)),
                                            ("conf", ref["conf"]), ("quaternion", ref["quaternion"]),
                                            ("translation", ref["translation"]))}
    agree = float(np.mean(out["mask"].astype(bool) == ref["mask"].numpy()))
    report(name, dtype=dtype, worst_block=f"{worst[1]:.7f}@{worst[0]}", depth_median_rel=f"{med:.2e}",
           mask_agree=f"{agree:.4f}", **{k + "_cos": f"{v:.7f}" for k, v in cos.items()})
    for b, c in res.items():
        assert c >= cos_min, ("block", b, c)
    assert med <= med_max
    for k, v in cos.items():
        assert v >= cos_min, (k, v)
    assert agree >= 0.99


def test_real_views_forward(ctx, views, weights):
    path, w = weights
    ref, rtaps = _oracle(w, views)
    for dtype in ("bf16", "f16"):
        _check("real_views.forward", ctx, path, dtype, views, ref, rtaps)


def test_real_views_known_cameras_f16(ctx, views, weights):
    path, w = weights
    intr = _intrinsics()
    ref, rtaps = _oracle(w, views, intrinsics=intr)
    _check("real_views.cameras", ctx, path, "f16", views, ref, rtaps, intrinsics=intr)
