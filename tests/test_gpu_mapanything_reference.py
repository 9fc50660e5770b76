"""MapAnything at the reference's own dims (mapanything-rs/src/dinov2.rs:8-10: ViT-giant width 1536,
24 heads, SwiGLU hidden 4096, 24 encoder blocks; info_sharing.rs:12-14: 16 alternating blocks at
1536, hooks after 7 and 11 and the last), the spec the real checkpoint needs. Loaded with a NULL
spec (splat_load_mapanything's reference constants) and compared with the CPU oracle on two small
views. The feed-forwards run the SwiGLU gate in the w12 GEMM's epilogue (mapanything-rs/src/
vit_block.rs:64-70; rows interleaved at load). LayerScale 1 so that every block changes the
residual stream. fp32: every block's stream at cosine >= 0.99999 and the outputs within 1e-3
relative error; bf16: every block at cosine >= 0.999 and the median depth error <= 1e-2.
The checkpoint has 1.2 G parameters (4.7 GB in fp32); generating it dominates the test's time.
"""
import gc
import os

import numpy as np
import pytest

from conftest import report, rel_err, cosine

pytestmark = [pytest.mark.gpu, pytest.mark.slow]

from splathip import specs, synth
from oracle import mapanything as O

SPEC = specs.MA_SPECS["reference"]


@pytest.fixture(scope="module")
def reference_weights(weights_dir):
    w = synth.generate(synth.ma_shapes(SPEC), seed=61, layer_scale=1.0)
    path = os.path.join(str(weights_dir), "ma_reference.safetensors")
    synth.save(path, w)
    yield path, w
    os.unlink(path)
    del w
    gc.collect()


def _run(ctx, path, dtype, images):
    ctx.load_mapanything(path, None, dtype)  # NULL spec: the reference constants
    taps = []
    ctx.set_debug_taps(lambda b, x: taps.append(x))
    try:
        out = ctx.ma_forward(images)
    finally:
        ctx.set_debug_taps(None)
    return out, taps


def test_ma_reference_dims_fp32(ctx, reference_weights):
    path, w = reference_weights
    images = synth.procedural_images(2, 42, 56, seed=62)
    report("ma.reference.fp32", views=2, hw="42x56", blocks=SPEC.enc_depth + SPEC.info_depth)
    out, taps = _run(ctx, path, "f32", images)
    enc_taps, info_taps = [], []
    ref = O.forward(w, SPEC, images, taps=enc_taps, info_taps=info_taps)
    rtaps = enc_taps + info_taps
    assert len(taps) == len(rtaps) == SPEC.enc_depth + SPEC.info_depth
    worst = min(cosine(a, b.reshape(a.shape).numpy()) for a, b in zip(taps, rtaps))
    errs = {
        "raw": rel_err(out["raw"], ref["raw"].numpy()),
        "quaternion": rel_err(out["quaternion"], ref["quaternion"].numpy()),
        "translation": rel_err(out["translation"], ref["translation"].numpy()),
        "scale": rel_err(out["scale"], [ref["scale"]], tau=0.0),
        "points": rel_err(out["points"], ref["points"].permute(0, 2, 3, 1).numpy()),
        "conf": rel_err(out["conf"], ref["conf"].numpy(), tau=0.0),
    }
    report("ma.reference.fp32.errs", worst_block_cos=f"{worst:.7f}", **{k: f"{v:.2e}" for k, v in errs.items()})
    assert worst > 0.99999
    for k, v in errs.items():
        assert v < 1e-3, (k, v)


def test_ma_reference_dims_bf16(ctx, reference_weights):
    path, w = reference_weights
    images = synth.procedural_images(2, 56, 42, seed=63)
    report("ma.reference.bf16", views=2, hw="56x42")
    out, taps = _run(ctx, path, "bf16", images)
    enc_taps, info_taps = [], []
    ref = O.forward(w, SPEC, images, taps=enc_taps, info_taps=info_taps)
    worst = min(cosine(a, b.reshape(a.shape).numpy()) for a, b in zip(taps, enc_taps + info_taps))
    depth = np.exp(out["raw"][:, 3].astype(np.float64)) * out["scale"][0]
    rdepth = np.exp(ref["raw"][:, 3].double().numpy()) * ref["scale"]
    med = float(np.median(np.abs(depth / rdepth - 1)))
    craw = cosine(out["raw"], ref["raw"].numpy())
    report("ma.reference.bf16.errs", worst_block_cos=f"{worst:.6f}", depth_median_rel=f"{med:.2e}",
           raw_cos=f"{craw:.6f}")
    assert worst >= 0.999
    assert med <= 1e-2
    assert craw >= 0.999
