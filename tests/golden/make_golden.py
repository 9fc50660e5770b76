"""Writes the golden fixtures of tests/golden/ from the CPU oracle (fp64 arithmetic, stored as
float32): seeded weights and images are regenerated from their seeds by splathip.synth, so a
fixture holds only the seeds, the configuration and the expected outputs.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "splatting-rs_amd")]

from oracle import da3 as OD  # noqa: E402
from oracle import mapanything as OM  # noqa: E402
from splathip import specs, synth  # noqa: E402

CASES = {
    "da3_small_3v_28x42": dict(model="da3", spec="small", views=3, h=28, w=42, wseed=31, iseed=32, ls=1.0),
    "ma_tiny_2v_28x42": dict(model="ma", spec="tiny", views=2, h=28, w=42, wseed=41, iseed=42, ls=1.0),
    "ma_tinyproj_2v_42x28": dict(model="ma", spec="tiny_proj", views=2, h=42, w=28, wseed=51, iseed=52, ls=1.0),
}


def case_inputs(c):
    if c["model"] == "da3":
        spec = specs.DA3_VARIANTS[c["spec"]]
        w = synth.generate(synth.da3_shapes(spec), seed=c["wseed"], layer_scale=c["ls"])
    else:
        spec = specs.MA_SPECS[c["spec"]]
        w = synth.generate(synth.ma_shapes(spec), seed=c["wseed"], layer_scale=c["ls"])
    images = synth.procedural_images(c["views"], c["h"], c["w"], seed=c["iseed"])
    return spec, w, images


def run_oracle(c, spec, w, images, dtype=torch.float64):
    if c["model"] == "da3":
        out = OD.forward_raw(w, spec, images, OD.REF_SADDLE, dtype=dtype)
        return {k: np.asarray(out[k], np.float32) for k in ("depth", "depth_conf", "ray_logits", "pose_encoding")} | \
            {"reference_view": np.int32(out["reference_view"])}
    out = OM.forward(w, spec, images, dtype=dtype)
    return {"raw": out["raw"].numpy().astype(np.float32), "quaternion": out["quaternion"].numpy().astype(np.float32),
            "translation": out["translation"].numpy().astype(np.float32), "scale": np.float32(out["scale"])}


def main():
    for name, c in CASES.items():
        spec, w, images = case_inputs(c)
        out = run_oracle(c, spec, w, images)
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **out)
        print(name, {k: v.shape for k, v in out.items()}, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
