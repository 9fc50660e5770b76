"""The drop-in boundary's remaining entry points, through the C ABI:

* the progress callback of splat_da3_forward_raw (DepthAnything3::forward_raw_with_progress,
  depthanything3-rs/src/model.rs:26-34,105-123; backbone.rs:156): Stage::Block(i) as each of
  the variant's blocks starts, then DenseHead, then CameraHead, on the calling thread; a
  forward with a callback runs eagerly even when graphs are on (a captured graph could not call
  back between stages) and gives the captured forward's outputs bit for bit;
* the in-memory checkpoint loaders (weights::model_from_safetensors_bytes,
  depthanything3-rs/src/weights.rs:51-60, which the browser worker calls with fetched bytes,
  web/src/reconstruct.rs:66-78; MapAnything's equivalent): the same outputs, bit for bit, as
  the file loaders.
"""
import os

import numpy as np
import pytest

from conftest import report

pytestmark = pytest.mark.gpu

import splathip
from splathip import specs, synth

DA3 = specs.DA3_VARIANTS["small"]
MA = specs.MA_SPECS["tiny"]
DA3_KEYS = ("depth", "depth_conf", "ray_logits", "pose_encoding", "camera_tokens")
MA_KEYS = ("raw", "quaternion", "translation", "scale", "points", "conf", "mask")


@pytest.fixture(scope="module")
def da3_path(weights_dir):
    path = os.path.join(str(weights_dir), "boundary_da3_small.safetensors")
    synth.save(path, synth.generate(synth.da3_shapes(DA3), seed=41, layer_scale=1.0))
    return path


@pytest.fixture(scope="module")
def ma_path(weights_dir):
    path = os.path.join(str(weights_dir), "boundary_ma_tiny.safetensors")
    synth.save(path, synth.generate(synth.ma_shapes(MA), seed=42, layer_scale=1.0))
    return path


def test_da3_progress_reports_every_stage_and_bypasses_graphs(ctx, da3_path):
    images = synth.procedural_images(3, 56, 42, seed=43)
    ctx.load_da3(da3_path, "small", "bf16", specs.REF_SADDLE)
    want = [(splathip.STAGE_BLOCK, i) for i in range(DA3.depth)]
    want += [(splathip.STAGE_DENSE_HEAD, 0), (splathip.STAGE_CAMERA_HEAD, 0)]
    ctx.set_graphs(True)
    try:
        captured = ctx.da3_forward_raw(images)       # captured into a graph, then replayed
        replayed = ctx.da3_forward_raw(images)
        runs = []
        for rep in range(2):
            stages = []
            out = ctx.da3_forward_raw(images, progress=lambda s, b: stages.append((s, b)))
            report("boundary.progress", rep=rep, stages=len(stages))
            runs.append((stages, out))
        after = ctx.da3_forward_raw(images)          # the graph again, without a callback
    finally:
        ctx.set_graphs(False)
    for stages, out in runs:
        assert stages == want
        for k in DA3_KEYS:
            assert np.array_equal(out[k], captured[k]), k
        assert out["reference_view"] == captured["reference_view"]
    for o in (replayed, after):
        for k in DA3_KEYS:
            assert np.array_equal(o[k], captured[k]), k


def test_da3_progress_without_graphs(ctx, da3_path):
    images = synth.procedural_images(4, 42, 56, seed=44)
    ctx.load_da3(da3_path, "small", "f32", specs.REF_SADDLE)
    plain = ctx.da3_forward_raw(images)
    stages = []
    out = ctx.da3_forward_raw(images, progress=lambda s, b: stages.append((s, b)))
    assert [s for s in stages if s[0] == splathip.STAGE_BLOCK] == [(splathip.STAGE_BLOCK, i) for i in range(DA3.depth)]
    assert stages[-2:] == [(splathip.STAGE_DENSE_HEAD, 0), (splathip.STAGE_CAMERA_HEAD, 0)]
    for k in DA3_KEYS:
        assert np.array_equal(out[k], plain[k]), k


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_da3_bytes_loader_matches_the_file_loader(ctx, da3_path, dtype):
    images = synth.procedural_images(3, 42, 56, seed=45)
    report("boundary.da3_bytes", dtype=dtype)
    ctx.load_da3(da3_path, "small", dtype, specs.REF_SADDLE)
    a = ctx.da3_forward_raw(images)
    with open(da3_path, "rb") as f:
        data = f.read()
    ctx.load_da3_bytes(data, "small", dtype, specs.REF_SADDLE)
    del data  # the library copied what it needs
    b = ctx.da3_forward_raw(images)
    for k in DA3_KEYS:
        assert np.array_equal(a[k], b[k]), k
    assert a["reference_view"] == b["reference_view"]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_mapanything_bytes_loader_matches_the_file_loader(ctx, ma_path, dtype):
    images = synth.procedural_images(2, 28, 42, seed=46)
    report("boundary.ma_bytes", dtype=dtype)
    ctx.load_mapanything(ma_path, MA, dtype)
    a = ctx.ma_forward(images)
    with open(ma_path, "rb") as f:
        data = f.read()
    ctx.load_mapanything_bytes(data, MA, dtype)
    del data
    b = ctx.ma_forward(images)
    for k in MA_KEYS:
        assert np.array_equal(a[k], b[k]), k


def test_bytes_loaders_reject_truncated_checkpoints(ctx, da3_path, ma_path):
    for path, load in ((da3_path, lambda d: ctx.load_da3_bytes(d, "small", "f32")),
                       (ma_path, lambda d: ctx.load_mapanything_bytes(d, MA, "f32"))):
        with open(path, "rb") as f:
            data = f.read()
        for cut in (0, 7, 64, len(data) // 2, len(data) - 1):
            with pytest.raises(splathip.SplatError) as e:
                load(data[:cut])
            assert e.value.code in (splathip.IO_ERROR, splathip.SHAPE_MISMATCH, splathip.MISSING_KEY), (path, cut)
