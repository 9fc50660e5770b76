"""MapAnything through the C ABI (splat_load_mapanything + splat_ma_forward / splat_ma_encode)
against the CPU oracle (oracle/mapanything.py) on identical seeded weights and images, for
small specs of the same topology (GELU and SwiGLU feed-forwards, with and without the
encoder->info projection). Tolerances as in test_gpu_da3.py."""
import os

import numpy as np
import pytest

from conftest import report, rel_err, cosine, H16

pytestmark = pytest.mark.gpu

import splathip
from splathip import specs, synth
from oracle import mapanything as O


@pytest.fixture(scope="module")
def ma_weights(weights_dir):
    out = {}
    for name in ("tiny", "tiny_proj"):
        for ls in (1e-5, 1.0):
            spec = specs.MA_SPECS[name]
            w = synth.generate(synth.ma_shapes(spec), seed=21, layer_scale=ls)
            path = os.path.join(str(weights_dir), f"ma_{name}_{ls}.safetensors")
            synth.save(path, w)
            out[(name, ls)] = (path, w, spec)
    return out


def _check_fp32(out, ref):
    errs = {
        "raw": rel_err(out["raw"], ref["raw"].numpy()),
        "quaternion": rel_err(out["quaternion"], ref["quaternion"].numpy()),
        "translation": rel_err(out["translation"], ref["translation"].numpy()),
        "scale": rel_err(out["scale"], [ref["scale"]], tau=0.0),
        "points": rel_err(out["points"], ref["points"].permute(0, 2, 3, 1).numpy()),
        "conf": rel_err(out["conf"], ref["conf"].numpy(), tau=0.0),
    }
    report("ma.fp32.errs", **{k: f"{v:.2e}" for k, v in errs.items()})
    for k, v in errs.items():
        assert v < 1e-3, (k, v)
    agree = np.mean(out["mask"].astype(bool) == ref["mask"].numpy())
    assert agree > 0.999


@pytest.mark.parametrize("name", ["tiny", "tiny_proj"])
@pytest.mark.parametrize("ls", [1e-5, 1.0])
def test_ma_tiny_fp32(ctx, ma_weights, name, ls):
    path, w, spec = ma_weights[(name, ls)]
    images = synth.procedural_images(3, 56, 70, seed=4)
    report("ma.tiny.fp32", spec=name, ls=ls)
    ctx.load_mapanything(path, spec, "f32")
    taps = []
    ctx.set_debug_taps(lambda b, x: taps.append(x))
    try:
        out = ctx.ma_forward(images)
    finally:
        ctx.set_debug_taps(None)
    enc_taps, info_taps = [], []
    ref = O.forward(w, spec, images, taps=enc_taps, info_taps=info_taps)
    _check_fp32(out, ref)
    rtaps = [t.reshape(-1, t.shape[-1]) for t in enc_taps + info_taps]
    assert len(taps) == len(rtaps)
    for i, (a, b) in enumerate(zip(taps, rtaps)):
        assert cosine(a, b.numpy()) > 0.99999, i


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("hw", [(56, 70), (224, 224)])
def test_ma_head_fused_16bit(ctx, weights_dir, hw, dtype):
    """The 256-feature DPT head in bf16 and f16: its 128-channel output convolution computes the
    1x1 head and dense_output in its epilogue (no stored map); outputs against the oracle. At
    3x224x224 (150k pixels) the convolution runs on the two-blocks-per-CU 192x128 tiles."""
    cos_min, med_max = H16[dtype]
    spec = specs.MA_SPECS["tiny_f256"]
    w = synth.generate(synth.ma_shapes(spec), seed=23, layer_scale=1.0)
    path = os.path.join(str(weights_dir), "ma_tiny_f256.safetensors")
    synth.save(path, w)
    images = synth.procedural_images(3, hw[0], hw[1], seed=9)
    report("ma.head_fused", dtype=dtype, hw=hw)
    ctx.load_mapanything(path, spec, dtype)
    out = ctx.ma_forward(images)
    ref = O.forward(w, spec, images)
    depth = np.exp(out["raw"][:, 3]) * out["scale"][0]
    rdepth = np.exp(ref["raw"][:, 3].numpy()) * ref["scale"]
    med = float(np.median(np.abs(depth / rdepth - 1)))
    craw = cosine(out["raw"], ref["raw"].numpy())
    cpts = cosine(out["points"], ref["points"].permute(0, 2, 3, 1).numpy())
    cconf = cosine(out["conf"], ref["conf"].numpy())
    agree = float(np.mean(out["mask"].astype(bool) == ref["mask"].numpy()))
    report("ma.head_fused.errs", depth_median_rel=f"{med:.2e}", raw_cos=f"{craw:.6f}", points_cos=f"{cpts:.6f}",
           conf_cos=f"{cconf:.6f}", mask_agree=f"{agree:.4f}")
    assert med <= med_max
    assert craw >= cos_min and cpts >= cos_min and cconf >= cos_min
    assert agree >= 0.99


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("name", ["tiny", "tiny_proj"])
def test_ma_tiny_16bit(ctx, ma_weights, name, dtype):
    cos_min, med_max = H16[dtype]
    path, w, spec = ma_weights[(name, 1.0)]
    images = synth.procedural_images(3, 56, 70, seed=8)
    report("ma.tiny", dtype=dtype, spec=name)
    ctx.load_mapanything(path, spec, dtype)
    taps = []
    ctx.set_debug_taps(lambda b, x: taps.append(x))
    try:
        out = ctx.ma_forward(images)
    finally:
        ctx.set_debug_taps(None)
    enc_taps, info_taps = [], []
    ref = O.forward(w, spec, images, taps=enc_taps, info_taps=info_taps)
    for i, (a, b) in enumerate(zip(taps, enc_taps + info_taps)):
        c = cosine(a, b.reshape(a.shape).numpy())
        report("ma.tiny.block", i=i, cos=f"{c:.7f}")
        assert c >= cos_min, (i, c)
    depth = np.exp(out["raw"][:, 3]) * out["scale"][0]
    rdepth = np.exp(ref["raw"][:, 3].numpy()) * ref["scale"]
    med = float(np.median(np.abs(depth / rdepth - 1)))
    report("ma.tiny.depth", median_rel=f"{med:.2e}")
    assert med <= med_max
    assert cosine(out["raw"], ref["raw"].numpy()) >= cos_min
    assert cosine(out["quaternion"], ref["quaternion"].numpy()) >= cos_min


def test_ma_encoder_only(ctx, ma_weights):
    path, w, spec = ma_weights[("tiny", 1.0)]
    images = synth.uniform_images(2, 42, 56, seed=3)
    ctx.load_mapanything(path, spec, "f32")
    tok = ctx.ma_encode(images)
    ref = O.forward(w, spec, images, encoder_only=True)["encoder_tokens"].numpy()
    assert rel_err(tok, ref) < 1e-3


def test_ma_views_equivariance(ctx, ma_weights):
    """Permuting views 1.. (view 0 carries the reference embedding) permutes every per-view
    output and leaves the scale unchanged (global attention is permutation-equivariant)."""
    path, w, spec = ma_weights[("tiny", 1.0)]
    images = synth.procedural_images(4, 42, 42, seed=12)
    ctx.load_mapanything(path, spec, "f32")
    a = ctx.ma_forward(images)
    perm = [0, 3, 1, 2]
    b = ctx.ma_forward(images[perm])
    assert rel_err(b["raw"], a["raw"][perm]) < 1e-4
    assert rel_err(b["scale"], a["scale"], tau=0.0) < 1e-5


def test_ma_errors(ctx, ma_weights):
    path, w, spec = ma_weights[("tiny", 1e-5)]
    cs = splathip.MaSpecC.from_spec(spec)
    # a dtype outside splat_dtype is refused
    assert ctx._lib.splat_load_mapanything(ctx.handle, path.encode(), splathip.C.byref(cs), 3) == splathip.BAD_ARGUMENT
    ctx.load_mapanything(path, spec, "f32")
    with pytest.raises(splathip.SplatError) as e:
        ctx.ma_forward(np.zeros((1, 3, 56, 69), np.float32))
    assert e.value.code == splathip.BAD_SHAPE
    bad = specs.MA_SPECS["tiny_proj"]
    with pytest.raises(splathip.SplatError) as e:
        ctx.load_mapanything(path, bad, "f32")
    assert e.value.code in (splathip.MISSING_KEY, splathip.SHAPE_MISMATCH)


# --- known cameras: the ray encoder (mapanything-rs/src/model.rs:97-102, ray_encoder.rs) -----

CAMS = [(60.0, 62.0, 34.5, 27.5), (48.0, 48.0, 30.0, 20.0), (90.0, 70.0, 10.0, 40.0)]


@pytest.mark.parametrize("known", [(0, 1, 2), (1,)])
def test_ma_known_cameras_fp32(ctx, ma_weights, known):
    path, w, spec = ma_weights[("tiny_proj", 1.0)]
    images = synth.procedural_images(3, 56, 70, seed=8)
    intr = [CAMS[v] if v in known else None for v in range(3)]
    report("ma.rays.fp32", known=known)
    ctx.load_mapanything(path, spec, "f32")
    out = ctx.ma_forward(images, intrinsics=intr)
    ref = O.forward(w, spec, images, intrinsics=intr)
    _check_fp32(out, ref)
    # the cameras change the result (the ray features are not lost on the way)
    plain = O.forward(w, spec, images)
    assert rel_err(ref["raw"].numpy(), plain["raw"].numpy()) > 1e-3


def test_ma_known_cameras_bf16_and_graph_replay(ctx, ma_weights):
    path, w, spec = ma_weights[("tiny", 1.0)]
    images = synth.procedural_images(3, 42, 56, seed=9)
    intr = [CAMS[0], None, CAMS[2]]
    ctx.load_mapanything(path, spec, "bf16")
    ref = O.forward(w, spec, images, intrinsics=intr)
    ctx.set_graphs(True)
    try:
        outs = [ctx.ma_forward(images, intrinsics=intr) for _ in range(3)]
        other = ctx.ma_forward(images, intrinsics=[CAMS[1], None, CAMS[0]])
        again = ctx.ma_forward(images, intrinsics=intr)
    finally:
        ctx.set_graphs(False)
    for o in outs + [again]:
        c = cosine(o["raw"], ref["raw"].numpy())
        report("ma.rays.bf16", cos_raw=f"{c:.6f}")
        assert c >= 0.999
        assert np.array_equal(o["raw"], outs[0]["raw"])
    # new camera values on the same captured graph are read at replay
    ref_other = O.forward(w, spec, images, intrinsics=[CAMS[1], None, CAMS[0]])
    assert cosine(other["raw"], ref_other["raw"].numpy()) >= 0.999
    assert not np.array_equal(other["raw"], outs[0]["raw"])


def test_ma_known_cameras_need_the_ray_encoder(ctx, ma_weights, weights_dir):
    path, w, spec = ma_weights[("tiny", 1e-5)]
    stripped = {k: v for k, v in w.items() if not k.startswith("ray_dirs_encoder.")}
    p2 = os.path.join(str(weights_dir), "ma_tiny_norays.safetensors")
    synth.save(p2, stripped)
    ctx.load_mapanything(p2, spec, "f32")
    images = synth.procedural_images(2, 28, 42, seed=1)
    a = ctx.ma_forward(images)                       # unknown cameras need no ray encoder
    b = ctx.ma_forward(images, intrinsics=[None, None])
    assert np.array_equal(a["raw"], b["raw"])
    with pytest.raises(splathip.SplatError) as e:
        ctx.ma_forward(images, intrinsics=[CAMS[0], None])
    assert e.value.code == splathip.MISSING_KEY
