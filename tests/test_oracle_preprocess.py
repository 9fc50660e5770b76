"""Pins of oracle/preprocess.py (the `image` crate's resize and both crates' input-size rules) by
the reference's own unit tests and by what the mathematics fixes; and the library's host-side size
functions (splat_da3_input_size, splat_ma_input_size: no GPU needed) against the oracle. CPU only.
"""
import math

import numpy as np
import pytest

import splathip
from oracle import preprocess as P

FILTERS = [P.TRIANGLE, P.CATMULLROM, P.LANCZOS3]


# --- known answers from the reference's tests ---------------------------------------------

def test_da3_sizes_known_answers():
    # depthanything3-rs/src/preprocess.rs:128-142
    assert P.model_input_size(3024, 4032) == ((378, 504), (378, 504))
    assert P.model_input_size(1920, 1080) == ((504, 284), (504, 280))
    assert P.nearest_multiple(377, 14) == 378
    assert P.nearest_multiple(371, 14) == 378
    assert P.nearest_multiple(370, 14) == 364


def test_ma_sizes_known_answers():
    # mapanything-rs/src/preprocess.rs:86-100
    assert P.input_size([(3024, 4032)]) == (392, 518)
    assert P.input_size([(1920, 1080)]) == (518, 294)
    (rw, rh), (left, top), _ = P.cover(1000, 700, (518, 392))
    assert rw >= 518 and rh >= 392 and 0 <= left <= rw - 518 and 0 <= top <= rh - 392
    img = np.zeros((700, 1000, 4), np.uint8)
    out = P.resize(img, rw, rh, P.LANCZOS3)[top:top + 392, left:left + 518]
    assert out.shape == (392, 518, 4)


def test_library_size_functions_match_the_oracle():
    for w, h in [(3024, 4032), (1920, 1080), (504, 378), (640, 480), (100, 60), (1, 1000), (4000, 3),
                 (503, 505), (518, 392), (392, 518)]:
        assert splathip.da3_model_input_size(w, h) == P.model_input_size(w, h), (w, h)
    for sizes in [[(3024, 4032)], [(1920, 1080)], [(1000, 700), (700, 1000)], [(518, 392)] * 6,
                  [(300, 600), (1200, 400), (640, 480)], [(1, 100)], [(100, 1)]]:
        assert splathip.ma_input_size(sizes) == P.input_size(sizes), sizes
    with pytest.raises(splathip.SplatError):
        splathip.da3_model_input_size(0, 10)


# --- the resize, by mathematics -------------------------------------------------------------

def test_same_size_is_a_copy():
    rng = np.random.default_rng(0)
    img = rng.integers(0, 256, (7, 9, 4), dtype=np.uint8)
    for f in FILTERS:
        assert np.array_equal(P.resize(img, 9, 7, f), img)


@pytest.mark.parametrize("f", FILTERS)
def test_weights_normalised_and_symmetric(f):
    for n_in, n_out in [(10, 4), (10, 23), (37, 37 * 3), (100, 13)]:
        taps = P.resize_taps(n_in, n_out, f)
        for o, (left, w) in enumerate(taps):
            assert abs(float(np.sum(w.astype(np.float64))) - 1.0) < 1e-5
            right = left + len(w)
            assert 0 <= left < right <= n_in
        # mirror symmetry away from the clamped edges: output o and n_out - 1 - o, as dense
        # weights over the input positions (a window may carry an extra zero-weight tap)
        def dense(o):
            left, w = taps[o]
            d = np.zeros(n_in)
            d[left:left + len(w)] = w
            return d, left > 0 and left + len(w) < n_in
        for o in range(n_out):
            (d1, in1), (d2, in2) = dense(o), dense(n_out - 1 - o)
            if in1 and in2:
                assert np.allclose(d1, d2[::-1], atol=1e-6), o


@pytest.mark.parametrize("f", FILTERS)
def test_constant_image_stays_constant(f):
    img = np.full((20, 30, 4), 173, np.uint8)
    img[..., 3] = 255
    for nw, nh in [(11, 7), (61, 45), (30, 9)]:
        out = P.resize(img, nw, nh, f)
        assert np.all(out[..., :3] == 173) and np.all(out[..., 3] == 255)


def test_triangle_halving_is_the_1331_average():
    """ratio 2: source support 2, taps 2x-1..2x+2 at distances 0.75, 0.25, 0.25, 0.75 -> weights
    (1, 3, 3, 1) / 8 along each axis (away from the edges)."""
    rng = np.random.default_rng(1)
    img = rng.integers(0, 256, (16, 24, 4), dtype=np.uint8)
    out = P.resize(img, 12, 8, P.TRIANGLE).astype(np.float64)
    k = np.array([1, 3, 3, 1]) / 8.0
    src = img.astype(np.float64)
    for y in range(1, 7):
        for x in range(1, 11):
            block = src[2 * y - 1:2 * y + 3, 2 * x - 1:2 * x + 3]
            ref = np.einsum("i,j,ijc->c", k, k, block)
            assert np.all(np.abs(out[y, x] - ref) <= 0.5 + 1e-3), (y, x)


def test_triangle_enlarging_interpolates_linearly():
    """ratio < 1: support 1, output x samples input (x + 0.5) * r - 0.5 by linear interpolation."""
    w = 10
    ramp = np.tile((np.arange(w) * 20).astype(np.uint8)[None, :, None], (3, 1, 4))
    out = P.resize(ramp, 25, 3, P.TRIANGLE)[1, :, 0].astype(np.float64)
    r = w / 25
    for x in range(25):
        c = (x + 0.5) * r - 0.5
        if 0 <= c <= w - 1:
            assert abs(out[x] - 20 * c) <= 0.5 + 1e-3, x


def test_catmullrom_reproduces_linear_ramps():
    """The Keys cubic (b = 0, c = 0.5) reproduces linear functions: its weights at integer offsets
    sum to one and have first moment equal to the sample position."""
    w = 16
    ramp = np.tile((np.arange(w) * 12).astype(np.uint8)[None, :, None], (3, 1, 4))
    out = P.resize(ramp, 2 * w, 3, P.CATMULLROM)[1, :, 0].astype(np.float64)
    for x in range(4, 2 * w - 4):
        c = (x + 0.5) / 2 - 0.5
        assert abs(out[x] - 12 * c) <= 0.5 + 1e-3, x


def test_kernels_closed_forms():
    assert P._kernel(P.TRIANGLE, 0.25) == np.float32(0.75)
    assert P._kernel(P.TRIANGLE, 1.0) == 0.0
    assert P._kernel(P.CATMULLROM, 0.0) == 1.0
    assert P._kernel(P.CATMULLROM, 1.0) == 0.0 and P._kernel(P.CATMULLROM, 2.0) == 0.0
    assert abs(P._kernel(P.CATMULLROM, 0.5) - 0.5625) < 1e-7          # (9/8 - 15/4 + 6)/6
    assert abs(P._kernel(P.CATMULLROM, 1.5) + 0.0625) < 1e-7          # (-81/8 + 135/4 - 36 + 12)/6
    assert P._kernel(P.LANCZOS3, 0.0) == 1.0
    assert abs(P._kernel(P.LANCZOS3, 0.5) - 6 / math.pi ** 2) < 1e-6  # sinc(1/2) sinc(1/6)
    assert abs(P._kernel(P.LANCZOS3, 1.0)) < 1e-6 and P._kernel(P.LANCZOS3, 3.0) == 0.0


@pytest.mark.parametrize("f", FILTERS)
def test_separable_passes_equal_the_2d_weighted_sum(f):
    """The two passes (f32, rows then columns) against one 2-D sum in f64 with the same taps:
    equal up to the u8 rounding."""
    rng = np.random.default_rng(2)
    img = rng.integers(0, 256, (13, 17, 4), dtype=np.uint8)
    nw, nh = 7, 29
    out = P.resize(img, nw, nh, f).astype(np.int32)
    rows, cols = P.resize_taps(13, nh, f), P.resize_taps(17, nw, f)
    src = img.astype(np.float64)
    for y, (t, wy) in enumerate(rows):
        for x, (l, wx) in enumerate(cols):
            v = np.einsum("i,j,ijc->c", wy.astype(np.float64), wx.astype(np.float64),
                          src[t:t + len(wy), l:l + len(wx)])
            ref = np.clip(np.floor(v + 0.5), 0, 255)
            assert np.all(np.abs(out[y, x] - ref) <= 1), (y, x)
