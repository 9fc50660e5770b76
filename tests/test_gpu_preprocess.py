"""The device preprocessing (include/splathip.h: splat_resize_rgba8, splat_da3_model_inputs,
splat_ma_model_inputs) against oracle/preprocess.py, the restatement of image 0.25.10's resize and
both crates' preprocess.rs. The device runs the crate's f32 weights (computed on the host as the
crate does) with every product and sum rounded on its own, so the outputs of all three filters
are bit-exact against the oracle (whose Lanczos3 sinc takes the C library's sinf, as the host
code and Rust's f32::sin do).
"""
import numpy as np
import pytest

from conftest import report

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

import splathip
from oracle import preprocess as P


def _image(h, w, seed):
    """Smooth colour field plus noise (so that resampling is not trivially exact) with an alpha
    channel that has transparent regions."""
    rng = np.random.default_rng(seed)
    y, x = np.mgrid[0:h, 0:w].astype(np.float64)
    img = np.empty((h, w, 4), np.uint8)
    for c in range(3):
        f = 127 + 100 * np.sin(x / (5 + 3 * c) + y / (7 + c)) + rng.normal(0, 12, (h, w))
        img[..., c] = np.clip(f, 0, 255).astype(np.uint8)
    img[..., 3] = np.where((x - w / 2) ** 2 + (y - h / 2) ** 2 < (0.45 * min(h, w)) ** 2, 255, rng.integers(0, 200, (h, w)))
    return img


RESIZE_CASES = [
    # (h, w, new_h, new_w, filter)
    (48, 64, 21, 30, P.TRIANGLE),      # shrink, non-integer ratios
    (48, 64, 24, 32, P.TRIANGLE),      # halving
    (30, 40, 77, 91, P.CATMULLROM),    # enlarge
    (30, 40, 18, 55, P.CATMULLROM),    # one axis each way
    (700, 1000, 392, 560, P.LANCZOS3),  # MapAnything's cover of a 1000x700 photo (560x392, cropped to 518)
    (37, 53, 90, 20, P.LANCZOS3),
    (4032 // 8, 3024 // 8, 504 // 2, 378 // 2, P.TRIANGLE),  # a DA3 shrink at an eighth of an iPhone photo
    (64, 48, 64, 48, P.LANCZOS3),      # same size: a copy
]


@pytest.mark.parametrize("h,w,nh,nw,f", RESIZE_CASES)
def test_resize_matches_the_oracle(ctx, h, w, nh, nw, f):
    report("resize", h=h, w=w, nh=nh, nw=nw, filter=f)
    img = _image(h, w, seed=h * 31 + w)
    got = ctx.resize_rgba8(img, nw, nh, f)
    ref = P.resize(img, nw, nh, f)
    diff = np.abs(got.astype(np.int32) - ref.astype(np.int32))
    report("resize.diff", max=int(diff.max()), n_diff=int((diff > 0).sum()), size=diff.size)
    assert diff.max() == 0


def _model_inputs(ctx, fn, images, H, W):
    n = len(images)
    out = torch.empty(n, 3, H, W, device="cuda")
    fg = torch.empty(n, H, W, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    hw = fn(images, out.data_ptr(), fg.data_ptr())
    ctx.synchronize()
    assert hw == (H, W)
    return out.cpu().numpy(), fg.cpu().numpy().astype(bool)


def test_da3_model_inputs_match_the_oracle(ctx):
    """Three photos of different sizes: two resizes each (bounded, then patch multiples), center
    crop to the smallest, normalisation (depthanything3-rs/src/preprocess.rs:86-123)."""
    images = [_image(300, 420, 1), _image(510, 380, 2), _image(200, 520, 3)]
    W, H = splathip.da3_model_inputs_size([(im.shape[1], im.shape[0]) for im in images])
    report("da3.model_inputs", H=H, W=W)
    got, fg = _model_inputs(ctx, ctx.da3_model_inputs_device, images, H, W)
    ref, rfg = P.da3_model_inputs(images)
    assert ref.shape == got.shape
    assert np.array_equal(got, ref) and np.array_equal(fg, rfg)


def test_ma_model_inputs_match_the_oracle(ctx):
    """Cover and crop to the size the mean aspect ratio picks, Lanczos3 to shrink and CatmullRom
    to enlarge (mapanything-rs/src/preprocess.rs:43-80)."""
    images = [_image(700, 1000, 4), _image(300, 360, 5), _image(600, 900, 6)]
    W, H = splathip.ma_input_size([(im.shape[1], im.shape[0]) for im in images])
    report("ma.model_inputs", H=H, W=W)
    got, fg = _model_inputs(ctx, ctx.ma_model_inputs_device, images, H, W)
    ref, rfg = P.ma_model_inputs(images)
    assert ref.shape == got.shape
    assert np.array_equal(got, ref) and np.array_equal(fg, rfg)


def test_preprocess_errors(ctx):
    with pytest.raises(splathip.SplatError) as e:
        ctx.resize_rgba8(np.zeros((4, 4, 4), np.uint8), 2, 2, 7)
    assert e.value.code == splathip.BAD_ARGUMENT


def test_fully_transparent_view_is_an_error(ctx):
    """mapanything-rs/src/image_input.rs:196-197 (to_model_input, both crates): a view with no
    pixel of alpha >= 128 after cropping is an error naming it; one pixel at 128 is enough."""
    ok = _image(60, 80, 8)
    clear = _image(60, 80, 9)
    clear[..., 3] = 127
    edge = clear.copy()
    edge[0, 0, 3] = 128
    out = torch.empty(2, 3, 60, 80, device="cuda")
    fg = torch.empty(2, 60, 80, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    with pytest.raises(splathip.SplatError) as e:
        ctx.to_model_input_device(np.stack([ok, clear]), out.data_ptr(), fg.data_ptr())
    assert e.value.code == splathip.BAD_ARGUMENT and "view 1" in str(e.value) and "transparent" in str(e.value)
    ctx.to_model_input_device(np.stack([ok, edge]), out.data_ptr(), fg.data_ptr())
    ctx.synchronize()
    assert int(fg[1].sum()) == 1
    for fn in (ctx.da3_model_inputs_device, ctx.ma_model_inputs_device):
        big = torch.empty(2, 3, 1024, 1024, device="cuda")
        with pytest.raises(splathip.SplatError) as e:
            fn([clear, ok], big.data_ptr(), 0)
        assert e.value.code == splathip.BAD_ARGUMENT and "view 0" in str(e.value)
