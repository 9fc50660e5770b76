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

// The resize weights in f32 as the crate evaluates them: every product and sum rounded on its
// own (no fused multiply-add), a.powi(3) as (a * a) * a.
#pragma clang fp contract(off)

namespace splat {

namespace {

float triangle_kernel(float x) {
  const float a = std::fabs(x);
  return a < 1.0f ? 1.0f - a : 0.0f;
}

// bc_cubic_spline(x, b = 0, c = 0.5): (12 - 9b - 6c) = 9, (-18 + 12b + 6c) = -15, (6 - 2b) = 6;
// (-b - 6c) = -3, (6b + 30c) = 15, (-12b - 48c) = -24, (8b + 24c) = 12; the sum over 6.
float catmullrom_kernel(float x) {
  const float a = std::fabs(x);
  const float a2 = a * a, a3 = a2 * a;
  float k;
  if (a < 1.0f) {
    const float t3 = 9.0f * a3, t2 = -15.0f * a2;
    k = (t3 + t2) + 6.0f;
  } else if (a < 2.0f) {
    const float t3 = -3.0f * a3, t2 = 15.0f * a2, t1 = -24.0f * a;
    k = ((t3 + t2) + t1) + 12.0f;
  } else {
    k = 0.0f;
  }
  return k / 6.0f;
}

float sinc(float t) {
  const float a = t * 3.14159265358979323846f;
  return t == 0.0f ? 1.0f : std::sin(a) / a;
}

float lanczos3_kernel(float x) { return std::fabs(x) < 3.0f ? sinc(x) * sinc(x / 3.0f) : 0.0f; }

float kernel_at(int filter, float x) {
  switch (filter) {
    case SPLAT_FILTER_TRIANGLE: return triangle_kernel(x);
    case SPLAT_FILTER_CATMULLROM: return catmullrom_kernel(x);
    default: return lanczos3_kernel(x);
  }
}

float kernel_support(int filter) {
  return filter == SPLAT_FILTER_TRIANGLE ? 1.0f : filter == SPLAT_FILTER_CATMULLROM ? 2.0f : 3.0f;
}

// depthanything3-rs/src/preprocess.rs:22-34
uint32_t round_half_up(double v) { return uint32_t(std::max(std::floor(v + 0.5), 1.0)); }
uint32_t nearest_multiple(uint32_t value, uint32_t step) {
  const uint32_t down = value / step * step, up = down + step;
  return std::max(up - value <= value - down ? up : down, step);
}

constexpr uint32_t DA3_PROCESS_RESOLUTION = 504;  // depthanything3-rs/src/variant.rs:13
constexpr uint32_t PATCH = 14;                     // variant.rs:9

// mapanything-rs/src/preprocess.rs:16-29
constexpr struct { double aspect; uint32_t w, h; } MA_SIZE_BY_ASPECT[10] = {
    {0.486, 252, 518}, {0.567, 294, 518}, {0.649, 336, 518}, {0.757, 392, 518}, {1.000, 518, 518},
    {1.321, 518, 392}, {1.542, 518, 336}, {1.762, 518, 294}, {2.056, 518, 252}, {3.083, 518, 168}};
constexpr double COVER_SCALE_EPS = 1e-8;  // preprocess.rs:31

}  // namespace

// sample.rs vertical_sample / horizontal_sample: the input range and normalised weights of every
// output coordinate along one axis of `in` -> `out` samples.
ResizeTapsHost resize_taps(int in, int out, int filter) {
  ResizeTapsHost t;
  const float ratio = float(in) / float(out);
  const float sratio = ratio < 1.0f ? 1.0f : ratio;
  const float src_support = kernel_support(filter) * sratio;
  std::vector<float> ws;
  for (int o = 0; o < out; ++o) {
    float input = (float(o) + 0.5f) * ratio;
    long left = long(std::floor(input - src_support));
    left = std::min(std::max(left, 0L), long(in) - 1);
    long right = long(std::ceil(input + src_support));
    right = std::min(std::max(right, left + 1), long(in));
    input = input - 0.5f;
    ws.clear();
    float sum = 0.0f;
    for (long i = left; i < right; ++i) {
      const float w = kernel_at(filter, (float(i) - input) / sratio);
      ws.push_back(w);
      sum += w;
    }
    t.first.push_back(int(left));
    t.count.push_back(int(right - left));
    t.offset.push_back(int(t.w.size()));
    for (float w : ws) t.w.push_back(w / sum);
  }
  return t;
}

void da3_model_input_size(int width, int height, int& bw, int& bh, int& dw, int& dh) {
  SPLAT_CHECK(width > 0 && height > 0, BAD_ARGUMENT, "image size");
  const uint32_t w = uint32_t(width), h = uint32_t(height), longest = std::max(w, h);
  const double scale = double(DA3_PROCESS_RESOLUTION) / double(longest);
  uint32_t b0 = w, b1 = h;
  if (longest != DA3_PROCESS_RESOLUTION) {
    b0 = round_half_up(double(w) * scale);
    b1 = round_half_up(double(h) * scale);
  }
  bw = int(b0);
  bh = int(b1);
  dw = int(nearest_multiple(b0, PATCH));
  dh = int(nearest_multiple(b1, PATCH));
}

// depthanything3-rs/src/preprocess.rs:47-57: no resampling at the same size; CatmullRom when
// either side grows, else Triangle.
int da3_resize_filter(int w, int h, int nw, int nh) {
  return (nw > w || nh > h) ? SPLAT_FILTER_CATMULLROM : SPLAT_FILTER_TRIANGLE;
}

void ma_input_size(int n, const int* widths, const int* heights, int& width, int& height) {
  SPLAT_CHECK(n > 0 && widths && heights, BAD_ARGUMENT, "no images");
  double mean = 0.0;
  for (int k = 0; k < n; ++k) {
    SPLAT_CHECK(widths[k] > 0 && heights[k] > 0, BAD_ARGUMENT, "image size");
    mean += double(widths[k]) / double(heights[k]);
  }
  mean /= double(n);
  int best = 0;  // the closest entry; ties go to the smaller ratio (strict <, in table order)
  for (int e = 0; e < 10; ++e)
    if (std::fabs(MA_SIZE_BY_ASPECT[e].aspect - mean) < std::fabs(MA_SIZE_BY_ASPECT[best].aspect - mean)) best = e;
  width = int(MA_SIZE_BY_ASPECT[best].w);
  height = int(MA_SIZE_BY_ASPECT[best].h);
}

void ma_cover(int w, int h, int width, int height, int& rw, int& rh, int& left, int& top, int& filter) {
  const double scale = std::max(double(width) / double(w), double(height) / double(h)) + COVER_SCALE_EPS;
  filter = scale < 1.0 ? SPLAT_FILTER_LANCZOS3 : SPLAT_FILTER_CATMULLROM;
  rw = int(std::floor(double(w) * scale));
  rh = int(std::floor(double(h) * scale));
  left = (rw - width) / 2;
  top = (rh - height) / 2;
}

namespace {

// Staging slots of the preprocessing (Context::staging_buffer).
enum { SLOT_SRC = 40, SLOT_A = 41, SLOT_B = 42, SLOT_TMP = 43, SLOT_ROWS = 44, SLOT_COLS = 45, SLOT_BATCH = 46 };

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
  to_model_input(c.ex, batch, n, ch, cw, images, foreground);
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
  to_model_input(c.ex, batch, n, th, tw, images, foreground);
  H = th;
  W = tw;
}

}  // namespace splat
