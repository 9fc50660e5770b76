// Image preprocessing of both crates on the device: the input-size rules
// (depthanything3-rs/src/preprocess.rs:22-45, mapanything-rs/src/preprocess.rs:16-63), the
// `image` crate's resize (image 0.25.10, Cargo.lock:2536-2539, imageops/sample.rs: resize,
// vertical_sample, horizontal_sample and the Triangle / CatmullRom / Lanczos3 kernels; the crate
// is not vendored, this restates its published algorithm), center crops and to_model_input
// (mapanything-rs/src/image_input.rs:195-216).
#include <algorithm>
#include <array>
#include <cmath>
#include <cstring>
#include <vector>

#include "runtime.h"

namespace splat {

namespace {

// Staging slots of the preprocessing (Context::staging_buffer).
enum { SLOT_SRC = 40, SLOT_A = 41, SLOT_B = 42, SLOT_TMP = 43, SLOT_ROWS = 44, SLOT_COLS = 45, SLOT_BATCH = 46,
       SLOT_FLAGS = 49 };

ResizeTaps upload_taps(Context& c, int slot, const ResizeTapsHost& t) {
  const size_t n = t.first.size(), nw = t.w.size();
  std::vector<char> buf(3 * n * sizeof(int) + nw * sizeof(float));
  std::memcpy(buf.data(), t.first.data(), n * sizeof(int));
  std::memcpy(buf.data() + n * sizeof(int), t.count.data(), n * sizeof(int));
  std::memcpy(buf.data() + 2 * n * sizeof(int), t.offset.data(), n * sizeof(int));
  std::memcpy(buf.data() + 3 * n * sizeof(int), t.w.data(), nw * sizeof(float));
  char* d = static_cast<char*>(c.staging_buffer(slot, buf.size()));
  SPLAT_HIP(hipMemcpyAsync(d, buf.data(), buf.size(), hipMemcpyHostToDevice, c.stream));
  SPLAT_HIP(hipStreamSynchronize(c.stream));  // `buf` is released on return
  ResizeTaps r;
  r.first = reinterpret_cast<const int*>(d);
  r.count = reinterpret_cast<const int*>(d + n * sizeof(int));
  r.offset = reinterpret_cast<const int*>(d + 2 * n * sizeof(int));
  r.w = reinterpret_cast<const float*>(d + 3 * n * sizeof(int));
  return r;
}

}  // namespace

void resize_device(Context& c, const uint8_t* src, int w, int h, uint8_t* dst, int nw, int nh, int filter) {
  SPLAT_CHECK(filter >= SPLAT_FILTER_TRIANGLE && filter <= SPLAT_FILTER_LANCZOS3, BAD_ARGUMENT, "resize filter");
  SPLAT_CHECK(w > 0 && h > 0 && nw > 0 && nh > 0, BAD_ARGUMENT, "resize sizes");
  if (w == nw && h == nh) {  // sample.rs resize: a copy at the same size
    SPLAT_HIP(hipMemcpyAsync(dst, src, size_t(w) * h * 4, hipMemcpyDeviceToDevice, c.stream));
    return;
  }
  const ResizeTaps rows = upload_taps(c, SLOT_ROWS, resize_taps(h, nh, filter));
  const ResizeTaps cols = upload_taps(c, SLOT_COLS, resize_taps(w, nw, filter));
  float* tmp = static_cast<float*>(c.staging_buffer(SLOT_TMP, size_t(nh) * w * 4 * sizeof(float)));
  resize_rgba8(c.ex, src, w, h, tmp, dst, nw, nh, rows, cols);
  SPLAT_HIP(hipStreamSynchronize(c.stream));  // the taps' staging is reused by the next resize
}

namespace {

// One host image to the device (slot SLOT_SRC), resized through `sizes` in turn (each with its
// filter), the last result left in `out`'s slot; returns the device pointer of the result.
const uint8_t* resize_chain(Context& c, const uint8_t* host, int w, int h, const std::vector<std::array<int, 3>>& steps) {
  uint8_t* cur = static_cast<uint8_t*>(c.staging_buffer(SLOT_SRC, size_t(w) * h * 4));
  SPLAT_HIP(hipMemcpyAsync(cur, host, size_t(w) * h * 4, hipMemcpyHostToDevice, c.stream));
  int slot = SLOT_A;
  for (const auto& s : steps) {
    if (s[0] == w && s[1] == h) continue;  // no resampling at the same size
    uint8_t* nxt = static_cast<uint8_t*>(c.staging_buffer(slot, size_t(s[0]) * s[1] * 4));
    resize_device(c, cur, w, h, nxt, s[0], s[1], s[2]);
    cur = nxt;
    w = s[0];
    h = s[1];
    slot = slot == SLOT_A ? SLOT_B : SLOT_A;
  }
  return cur;
}

void crop_into(Context& c, const uint8_t* src, int w, int left, int top, int cw, int ch, uint8_t* dst) {
  SPLAT_HIP(hipMemcpy2DAsync(dst, size_t(cw) * 4, src + (size_t(top) * w + left) * 4, size_t(w) * 4, size_t(cw) * 4,
                             size_t(ch), hipMemcpyDeviceToDevice, c.stream));
}

}  // namespace

void model_input(Context& c, const uint8_t* rgba, int V, int H, int W, float* images, uint8_t* foreground) {
  int* flags = static_cast<int*>(c.staging_buffer(SLOT_FLAGS, size_t(V) * sizeof(int)));
  to_model_input(c.ex, rgba, V, H, W, images, foreground);
  foreground_any(c.ex, rgba, V, H, W, flags);
  std::vector<int> any(V);
  SPLAT_HIP(hipMemcpyAsync(any.data(), flags, size_t(V) * sizeof(int), hipMemcpyDeviceToHost, c.stream));
  SPLAT_HIP(hipStreamSynchronize(c.stream));
  for (int v = 0; v < V; ++v)  // image_input.rs:197 ensure!
    SPLAT_CHECK(any[v] != 0, BAD_ARGUMENT, "view " + std::to_string(v) + " is fully transparent after cropping");
}

void da3_model_inputs(Context& c, int n, const uint8_t* const* rgba, const int* widths, const int* heights, float* images,
                      uint8_t* foreground, int& H, int& W) {
  SPLAT_CHECK(n > 0 && rgba && widths && heights && images, BAD_ARGUMENT, "model_inputs args");
  std::vector<std::array<int, 4>> sz(n);
  int cw = 1 << 30, ch = 1 << 30;
  for (int k = 0; k < n; ++k) {
    SPLAT_CHECK(rgba[k] != nullptr, BAD_ARGUMENT, "model_inputs: missing image");
    da3_model_input_size(widths[k], heights[k], sz[k][0], sz[k][1], sz[k][2], sz[k][3]);
    cw = std::min(cw, sz[k][2]);
    ch = std::min(ch, sz[k][3]);
  }
  uint8_t* batch = static_cast<uint8_t*>(c.staging_buffer(SLOT_BATCH, size_t(n) * cw * ch * 4));
  for (int k = 0; k < n; ++k) {
    // preprocess.rs:59-64 resize_for_model: to the bounded size, then to the patch multiples
    const int w = widths[k], h = heights[k];
    std::vector<std::array<int, 3>> steps = {{sz[k][0], sz[k][1], da3_resize_filter(w, h, sz[k][0], sz[k][1])},
                                             {sz[k][2], sz[k][3], da3_resize_filter(sz[k][0], sz[k][1], sz[k][2], sz[k][3])}};
    const uint8_t* r = resize_chain(c, rgba[k], w, h, steps);
    // preprocess.rs:67-72 center_crop to the common size
    crop_into(c, r, sz[k][2], (sz[k][2] - cw) / 2, (sz[k][3] - ch) / 2, cw, ch, batch + size_t(k) * cw * ch * 4);
    SPLAT_HIP(hipStreamSynchronize(c.stream));  // the staging of this image is reused by the next
  }
  model_input(c, batch, n, ch, cw, images, foreground);
  H = ch;
  W = cw;
}

void ma_model_inputs(Context& c, int n, const uint8_t* const* rgba, const int* widths, const int* heights, float* images,
                     uint8_t* foreground, int& H, int& W) {
  SPLAT_CHECK(n > 0 && rgba && widths && heights && images, BAD_ARGUMENT, "model_inputs args");
  int tw, th;
  ma_input_size(n, widths, heights, tw, th);
  uint8_t* batch = static_cast<uint8_t*>(c.staging_buffer(SLOT_BATCH, size_t(n) * tw * th * 4));
  for (int k = 0; k < n; ++k) {
    SPLAT_CHECK(rgba[k] != nullptr, BAD_ARGUMENT, "model_inputs: missing image");
    int rw, rh, left, top, filter;
    ma_cover(widths[k], heights[k], tw, th, rw, rh, left, top, filter);
    const uint8_t* r = resize_chain(c, rgba[k], widths[k], heights[k], {{rw, rh, filter}});
    crop_into(c, r, rw, left, top, tw, th, batch + size_t(k) * tw * th * 4);
    SPLAT_HIP(hipStreamSynchronize(c.stream));
  }
  model_input(c, batch, n, th, tw, images, foreground);
  H = th;
  W = tw;
}

}  // namespace splat
