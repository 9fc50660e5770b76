"""The C-ABI library without a GPU: it loads, exports every symbol the public headers declare,
the Python binding types all of them, the reference spec matches, and host-side helpers
(synthetic checkpoints, specs) are consistent. No compute call is made here."""
import ctypes
import os
import re

import numpy as np
import pytest

import splathip
from splathip import specs, synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", f) for f in sorted(os.listdir(os.path.join(ROOT, "include"))) if f.endswith(".h")]


def declared_symbols():
    names = set()
    for h in HEADERS:
        text = open(h).read()
        names |= set(re.findall(r"^\s*(?:int|void|const char\s*\*|void\s*\*)\s*\**\s*(splat_\w+)\s*\(", text, re.M))
    return names


def test_headers_declare_the_entry_points():
    names = declared_symbols()
    for required in ("splat_create", "splat_destroy", "splat_load_da3", "splat_da3_forward_raw",
                     "splat_load_mapanything", "splat_ma_forward", "splat_last_error", "splat_set_debug_taps"):
        assert required in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(splathip.LIB_PATH)
    missing = [n for n in sorted(declared_symbols()) if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_types_every_declared_symbol():
    assert declared_symbols() == set(splathip.SIGNATURES)
    splathip.lib()


def test_reference_spec_matches_the_reference_constants():
    s = splathip.reference_ma_spec()
    r = specs.MA_SPECS["reference"]
    assert (s["enc_dim"], s["enc_heads"], s["enc_depth"], s["enc_hidden"]) == (r.enc_dim, r.enc_heads, r.enc_depth, r.enc_hidden)
    assert (s["info_dim"], s["info_depth"], s["hooks"]) == (r.info_dim, r.info_depth, list(r.hooks))
    assert s["dpt_dims"] == list(r.dpt_dims) and s["pose_dim"] == 784 and s["scale_dim"] == 196


def test_create_without_a_gpu_reports_an_error():
    torch = pytest.importorskip("torch")
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    h = ctypes.c_void_p()
    rc = splathip.lib().splat_create(0, ctypes.byref(h))
    assert rc == splathip.HIP_ERROR
    assert splathip.lib().splat_last_error(None)


def test_synthetic_checkpoint_is_seeded_per_tensor():
    shapes = synth.da3_shapes(specs.DA3_VARIANTS["small"])
    a = synth.generate(shapes, seed=7)
    b = synth.generate({k: shapes[k] for k in list(shapes)[::-1]}, seed=7, threads=1)
    assert all(np.array_equal(a[k], b[k]) for k in shapes)
    c = synth.generate(shapes, seed=8)
    assert not np.array_equal(a["model.head.norm.weight"], c["model.head.norm.weight"])
    assert np.all(a["model.backbone.pretrained.blocks.0.ls1.gamma"] == np.float32(1e-5))
    assert abs(float(a["model.head.norm.weight"].mean()) - 1.0) < 0.01


def test_checkpoint_key_maps():
    da3 = synth.da3_shapes(specs.DA3_VARIANTS["small"])
    assert da3["model.backbone.pretrained.pos_embed"][0] == (1, 1370, 384)
    assert "model.backbone.pretrained.blocks.3.attn.q_norm.weight" not in da3   # qk-norm from alt_start
    assert "model.backbone.pretrained.blocks.4.attn.q_norm.weight" in da3
    assert da3["model.head.resize_layers.0.weight"][0] == (48, 48, 4, 4)
    assert "model.head.scratch.refinenet4.resConfUnit1.conv1.weight" not in da3
    ma = synth.ma_shapes(specs.MA_SPECS["baseline_l"])
    assert ma["info_sharing.proj_embed.weight"][0] == (768, 1024)
    assert ma["dense_head.0.input_process.0.0.0.weight"][0] == (96, 1024, 1, 1)
    assert ma["dense_head.0.input_process.1.0.0.weight"][0] == (192, 768, 1, 1)
    assert "dense_head.0.input_process.2.0.1.weight" not in ma
    assert ma["ray_dirs_encoder.conv_in.weight"][0] == (588, 588, 3, 3)
    assert ma["ray_dirs_encoder.encoder.1.conv2.weight"][0] == (1024, 1024, 3, 3)
    assert ma["ray_dirs_encoder.encoder.2.weight"][0] == (1024, 1024, 1, 1)
    n = sum(int(np.prod(s)) for s, _ in ma.values())
    nray = sum(int(np.prod(s)) for k, (s, _) in ma.items() if k.startswith("ray_dirs_encoder."))
    assert 480e6 < n - nray < 520e6 and 31e6 < nray < 32e6


def test_configs_match_the_benchmark_table():
    c = specs.CONFIGS
    assert (c["C2"].views * ((c["C2"].height // 14) * (c["C2"].width // 14) + 1)) == 5838
    assert (c["C4"].views * ((c["C4"].height // 14) * (c["C4"].width // 14) + 1) + 1) == 6223
    assert (c["C5"].views * ((c["C5"].height // 14) * (c["C5"].width // 14) + 1) + 1) == 24889
    for cfg in c.values():
        assert cfg.height % 14 == 0 and cfg.width % 14 == 0


def test_procedural_images_are_normalised_and_seeded():
    a = synth.procedural_images(2, 28, 42, seed=1)
    b = synth.procedural_images(2, 28, 42, seed=1)
    assert np.array_equal(a, b) and a.shape == (2, 3, 28, 42) and a.dtype == np.float32
    rgb = a * np.asarray(specs.IMAGENET_STD, np.float32).reshape(1, 3, 1, 1) + np.asarray(specs.IMAGENET_MEAN, np.float32).reshape(1, 3, 1, 1)
    assert rgb.min() >= -1e-6 and rgb.max() <= 1 + 1e-6
