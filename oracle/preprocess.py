"""CPU oracle for the image preprocessing — TEST INFRASTRUCTURE ONLY (see oracle/common.py).

Restates, in numpy float32 with the same operation order, what both crates do to a decoded RGBA
image before the network:

* the `image` crate's resize (image 0.25.10, /root/reference/Cargo.lock:2536-2539; the crate
  is not vendored, so this follows its published imageops/sample.rs: `resize` samples rows
  (`vertical_sample`, f32 RGBA) then columns (`horizontal_sample`, rounded half away from zero
  and clamped to u8), each output coordinate weighting the inputs in [left, right) by the
  filter kernel at (i - (x + 0.5) * ratio + 0.5) / max(ratio, 1), normalised by their f32 sum;
  a copy at the same size), with the Triangle, CatmullRom (bc_cubic_spline b = 0, c = 0.5) and
  Lanczos3 kernels the crates use (depthanything3-rs/src/preprocess.rs:19-20,
  mapanything-rs/src/preprocess.rs:46-51);
* depthanything3-rs/src/preprocess.rs:22-123 (model_input_size, resize_exact, resize_for_model,
  center_crop to the common size) and mapanything-rs/src/preprocess.rs:16-80 (input_size,
  cover_and_crop), then to_model_input (oracle/common.py).

Pinned (tests/test_oracle_preprocess.py) by the reference's own unit tests of the sizes
(preprocess.rs tests of both crates) and by what the mathematics fixes for the resize: a copy
at the same size, constant images stay constant, a Triangle halving averages with weights
(1, 3, 3, 1) / 8, Triangle enlarging interpolates linearly, CatmullRom reproduces linear ramps,
every filter's weights sum to one and are symmetric, the separable passes equal the 2-D
weighted sum. What only the crate itself could pin (its exact f32 rounding sequence) is
"parity unpinned"; the restatement follows the published source's order. The Lanczos3 sinc takes
its sine from the C library's `sinf`, which is what Rust's `f32::sin` calls on Linux (and what the
library's host code calls), not numpy's float32 `np.sin`, whose vectorised routine differs from it
in the last bit for some arguments.
"""
import ctypes
import ctypes.util
import math

import numpy as np

from .common import to_model_input

TRIANGLE, CATMULLROM, LANCZOS3 = 1, 2, 3
_LIBM = ctypes.CDLL(ctypes.util.find_library("m") or "libm.so.6")
_sinf = _LIBM.sinf
_sinf.restype = ctypes.c_float
_sinf.argtypes = [ctypes.c_float]
_SUPPORT = {TRIANGLE: 1.0, CATMULLROM: 2.0, LANCZOS3: 3.0}
F = np.float32


def _kernel(filter_type, x):
    """The crate's kernels in float32 (sample.rs triangle_kernel, catmullrom_kernel via
    bc_cubic_spline(x, 0, 0.5), lanczos3_kernel via sinc): one value."""
    x = F(x)
    a = F(abs(x))
    if filter_type == TRIANGLE:
        return F(F(1.0) - a) if a < F(1.0) else F(0.0)
    if filter_type == CATMULLROM:
        a2 = F(a * a)
        a3 = F(a2 * a)
        if a < F(1.0):
            k = F(F(F(F(9.0) * a3) + F(F(-15.0) * a2)) + F(6.0))
        elif a < F(2.0):
            k = F(F(F(F(F(-3.0) * a3) + F(F(15.0) * a2)) + F(F(-24.0) * a)) + F(12.0))
        else:
            k = F(0.0)
        return F(k / F(6.0))

    def sinc(t):
        t = F(t)
        s = F(t * F(math.pi))
        return F(1.0) if t == F(0.0) else F(F(_sinf(s)) / s)

    return F(sinc(x) * sinc(F(x / F(3.0)))) if a < F(3.0) else F(0.0)


def resize_taps(n_in: int, n_out: int, filter_type: int):
    """sample.rs vertical_sample / horizontal_sample: (left, weights) of every output coordinate."""
    ratio = F(F(n_in) / F(n_out))
    sratio = F(1.0) if ratio < F(1.0) else ratio
    src_support = F(F(_SUPPORT[filter_type]) * sratio)
    taps = []
    for o in range(n_out):
        x = F(F(F(o) + F(0.5)) * ratio)
        left = int(math.floor(F(x - src_support)))
        left = min(max(left, 0), n_in - 1)
        right = int(math.ceil(F(x + src_support)))
        right = min(max(right, left + 1), n_in)
        x = F(x - F(0.5))
        ws, s = [], F(0.0)
        for i in range(left, right):
            w = _kernel(filter_type, F(F(F(i) - x) / sratio))
            ws.append(w)
            s = F(s + w)
        taps.append((left, np.array([F(w / s) for w in ws], F)))
    return taps


def resize(rgba: np.ndarray, new_w: int, new_h: int, filter_type: int) -> np.ndarray:
    """image::imageops::resize of an RGBA8 [h, w, 4] image (DynamicImage::resize_exact)."""
    h, w, _ = rgba.shape
    if (w, h) == (new_w, new_h):
        return rgba.copy()
    src = rgba.astype(F)
    tmp = np.zeros((new_h, w, 4), F)
    for y, (top, ws) in enumerate(resize_taps(h, new_h, filter_type)):
        acc = np.zeros((w, 4), F)
        for i, wt in enumerate(ws):
            acc = acc + src[top + i] * wt   # float32: product, then sum, rounded each
        tmp[y] = acc
    out = np.zeros((new_h, new_w, 4), np.uint8)
    for x, (left, ws) in enumerate(resize_taps(w, new_w, filter_type)):
        acc = np.zeros((new_h, 4), F)
        for i, wt in enumerate(ws):
            acc = acc + tmp[:, left + i] * wt
        v = np.clip(acc, F(0.0), F(255.0))
        out[:, x] = np.where(v >= 0, np.floor(v + F(0.5)), np.ceil(v - F(0.5))).astype(np.uint8)  # round half away
    return out


# --- Depth Anything 3 (depthanything3-rs/src/preprocess.rs) --------------------------------

PROCESS_RESOLUTION = 504   # depthanything3-rs/src/variant.rs:13
PATCH_SIZE = 14            # variant.rs:9


def _round_half_up(v: float) -> int:          # preprocess.rs:22-25
    return int(max(math.floor(v + 0.5), 1.0))


def nearest_multiple(value: int, step: int) -> int:   # preprocess.rs:27-32
    down = value // step * step
    up = down + step
    return max(up if up - value <= value - down else down, step)


def model_input_size(width: int, height: int):        # preprocess.rs:34-45
    longest = max(width, height)
    scale = PROCESS_RESOLUTION / longest
    bounded = (width, height) if longest == PROCESS_RESOLUTION else (_round_half_up(width * scale),
                                                                     _round_half_up(height * scale))
    return bounded, (nearest_multiple(bounded[0], PATCH_SIZE), nearest_multiple(bounded[1], PATCH_SIZE))


def _resize_exact_da3(rgba, w, h):                    # preprocess.rs:47-57
    ih, iw, _ = rgba.shape
    if (iw, ih) == (w, h):
        return rgba.copy()
    return resize(rgba, w, h, CATMULLROM if (w > iw or h > ih) else TRIANGLE)


def da3_model_inputs(images):
    """preprocess.rs:86-123 model_inputs_from_cutouts after decoding: list of RGBA8 [h, w, 4] ->
    (normalised images [n, 3, H, W] float32, foreground [n, H, W] bool)."""
    resized = []
    for im in images:
        bounded, divisible = model_input_size(im.shape[1], im.shape[0])
        resized.append(_resize_exact_da3(_resize_exact_da3(im, *bounded), *divisible))
    cw = min(r.shape[1] for r in resized)
    ch = min(r.shape[0] for r in resized)
    crops = []
    for r in resized:                                  # preprocess.rs:67-72 center_crop
        left, top = (r.shape[1] - cw) // 2, (r.shape[0] - ch) // 2
        crops.append(r[top:top + ch, left:left + cw])
    return to_model_input(np.stack(crops))


# --- MapAnything (mapanything-rs/src/preprocess.rs) ------------------------------------------

SIZE_BY_ASPECT = [(0.486, (252, 518)), (0.567, (294, 518)), (0.649, (336, 518)), (0.757, (392, 518)),
                  (1.000, (518, 518)), (1.321, (518, 392)), (1.542, (518, 336)), (1.762, (518, 294)),
                  (2.056, (518, 252)), (3.083, (518, 168))]   # preprocess.rs:16-29
COVER_SCALE_EPS = 1e-8                                         # preprocess.rs:31


def input_size(sizes):                                # preprocess.rs:33-41; sizes: [(w, h)]
    mean = sum(w / h for w, h in sizes) / len(sizes)
    best = SIZE_BY_ASPECT[0]
    for entry in SIZE_BY_ASPECT:
        if abs(entry[0] - mean) < abs(best[0] - mean):
            best = entry
    return best[1]


def cover(width, height, target):                     # preprocess.rs:43-63 (sizes and filter)
    tw, th = target
    scale = max(tw / width, th / height) + COVER_SCALE_EPS
    f = LANCZOS3 if scale < 1.0 else CATMULLROM
    rw, rh = int(math.floor(width * scale)), int(math.floor(height * scale))
    return (rw, rh), ((rw - tw) // 2, (rh - th) // 2), f


def ma_model_inputs(images):
    """preprocess.rs:66-80 load_images after decoding: list of RGBA8 [h, w, 4] -> (normalised
    images [n, 3, H, W] float32, foreground [n, H, W] bool)."""
    tw, th = input_size([(im.shape[1], im.shape[0]) for im in images])
    crops = []
    for im in images:
        (rw, rh), (left, top), f = cover(im.shape[1], im.shape[0], (tw, th))
        r = resize(im, rw, rh, f)
        crops.append(r[top:top + th, left:left + tw])
    return to_model_input(np.stack(crops))
