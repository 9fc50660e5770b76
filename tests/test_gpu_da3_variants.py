"""Depth Anything 3 Base, Large and Giant (variant.rs:73-113) through the C ABI against the CPU
oracle. Same checks as the Small tests (fp32: outputs within 1e-3 relative error and every
block's residual stream at cosine >= 0.99999; bf16: median depth error <= 1e-2), at LayerScale
1.0 so that every block changes the stream. Giant exercises the SwiGLU feed-forward
(w3(silu(x1) * x2), hidden swiglu_hidden_dim(1536) = 4096) and its 40-block alternation
(alt_start 13, hooks 19/27/33/39). Small images keep the oracle fast; the per-variant work is
mostly generating and loading the synthetic checkpoint (Giant: 1.1 G parameters).
"""
import gc
import os

import numpy as np
import pytest

from conftest import report, rel_err, cosine

pytestmark = [pytest.mark.gpu, pytest.mark.slow]

from splathip import specs, synth
from oracle import da3 as O


def _weights(variant, weights_dir, seed):
    spec = specs.DA3_VARIANTS[variant]
    w = synth.generate(synth.da3_shapes(spec), seed=seed, layer_scale=1.0)
    path = os.path.join(str(weights_dir), f"da3_{variant}.safetensors")
    synth.save(path, w)
    return spec, path, w


@pytest.mark.parametrize("variant", ["base", "large", "giant"])
def test_da3_variant_fp32(ctx, weights_dir, variant):
    spec, path, w = _weights(variant, weights_dir, seed=21)
    images = synth.procedural_images(3, 28, 42, seed=3)
    report("da3.variant.fp32", variant=variant, dim=spec.dim, depth=spec.depth, views=3, hw="28x42")
    taps = []
    ctx.load_da3(path, variant, "f32", specs.REF_SADDLE)
    ctx.set_debug_taps(lambda b, x: taps.append(x))
    try:
        out = ctx.da3_forward_raw(images)
    finally:
        ctx.set_debug_taps(None)
    rtaps = []
    ref = O.forward_raw(w, spec, images, specs.REF_SADDLE, taps=rtaps)
    errs = {
        "depth": rel_err(out["depth"], ref["depth"].numpy(), tau=0.0),
        "depth_conf": rel_err(out["depth_conf"], ref["depth_conf"].numpy(), tau=0.0),
        "ray_logits": rel_err(out["ray_logits"], ref["ray_logits"].numpy()),
        "pose_encoding": rel_err(out["pose_encoding"], ref["pose_encoding"].numpy()),
        "camera_tokens": rel_err(out["camera_tokens"], ref["camera_tokens"].numpy()),
    }
    report("da3.variant.fp32.errs", variant=variant, **{k: f"{v:.2e}" for k, v in errs.items()})
    for k, v in errs.items():
        assert v < 1e-3, (variant, k, v)
    assert out["reference_view"] == ref["reference_view"]
    assert len(taps) == len(rtaps) == spec.depth
    worst = min(cosine(a, b.reshape(a.shape).numpy()) for a, b in zip(taps, rtaps))
    report("da3.variant.fp32.blocks", variant=variant, min_cos=f"{worst:.7f}")
    assert worst > 0.99999
    del w, ref, taps, rtaps
    os.unlink(path)
    gc.collect()


def test_da3_giant_bf16(ctx, weights_dir):
    spec, path, w = _weights("giant", weights_dir, seed=22)
    images = synth.procedural_images(2, 42, 28, seed=4)
    report("da3.variant.bf16", variant="giant", views=2, hw="42x28")
    ctx.load_da3(path, "giant", "bf16", specs.REF_FIRST)
    out = ctx.da3_forward_raw(images)
    ref = O.forward_raw(w, spec, images, specs.REF_FIRST)
    med = float(np.median(np.abs(out["depth"] / ref["depth"].numpy() - 1)))
    c_ray = cosine(out["ray_logits"], ref["ray_logits"].numpy())
    c_pose = cosine(out["pose_encoding"], ref["pose_encoding"].numpy())
    report("da3.variant.bf16.errs", median_depth=f"{med:.2e}", cos_ray=f"{c_ray:.6f}", cos_pose=f"{c_pose:.6f}")
    assert med <= 1e-2
    assert c_ray >= 0.999 and c_pose >= 0.999
    del w, ref
    os.unlink(path)
    gc.collect()
