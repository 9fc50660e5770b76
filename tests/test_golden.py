"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py from the fp64
oracle): the fp32 oracle must reproduce them (CPU) and so must the HIP library (GPU)."""
import os
import sys

import numpy as np
import pytest

from conftest import rel_err, report

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_golden as G  # noqa: E402


def _load(name):
    with np.load(os.path.join(HERE, "golden", name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _compare(out, gold, tol):
    for k, v in gold.items():
        if k == "reference_view":
            assert int(out[k]) == int(v)
            continue
        tau = 0.0 if k in ("depth", "depth_conf", "scale") else 0.01
        e = rel_err(out[k], v, tau=tau)
        report("golden", key=k, err=f"{e:.2e}")
        assert e < tol, (k, e)


@pytest.mark.parametrize("name", sorted(G.CASES))
def test_fp32_oracle_reproduces_fixture(name):
    import torch
    c = G.CASES[name]
    spec, w, images = G.case_inputs(c)
    out = G.run_oracle(c, spec, w, images, dtype=torch.float32)
    _compare(out, _load(name), 1e-4)


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(G.CASES))
def test_library_reproduces_fixture(ctx, name, weights_dir):
    from splathip import synth
    c = G.CASES[name]
    spec, w, images = G.case_inputs(c)
    path = os.path.join(str(weights_dir), name + ".safetensors")
    synth.save(path, w)
    report("golden.gpu", case=name)
    if c["model"] == "da3":
        ctx.load_da3(path, c["spec"], "f32")
        out = ctx.da3_forward_raw(images)
    else:
        ctx.load_mapanything(path, spec, "f32")
        o = ctx.ma_forward(images)
        out = {"raw": o["raw"], "quaternion": o["quaternion"], "translation": o["translation"], "scale": o["scale"][0]}
    _compare(out, _load(name), 1e-3)
