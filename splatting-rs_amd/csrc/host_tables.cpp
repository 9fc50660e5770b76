// Host-side tables and size rules of the network path, in plain C++ (no HIP: the sanitizer test
// builds this file with a host compiler): the bicubic positional-embedding resize, the RoPE and
// uv-embedding tables, and the image preprocessing's size rules and resize taps.
#include "host_tables.h"

#include <algorithm>
#include <array>
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

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
  SPLAT_CHECK(in > 0 && out > 0, BAD_ARGUMENT, "resize sizes");
  SPLAT_CHECK(filter >= SPLAT_FILTER_TRIANGLE && filter <= SPLAT_FILTER_LANCZOS3, BAD_ARGUMENT, "resize filter");
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
  SPLAT_CHECK(w > 0 && h > 0 && width > 0 && height > 0, BAD_ARGUMENT, "image size");
  const double scale = std::max(double(width) / double(w), double(height) / double(h)) + COVER_SCALE_EPS;
  filter = scale < 1.0 ? SPLAT_FILTER_LANCZOS3 : SPLAT_FILTER_CATMULLROM;
  const double fw = std::floor(double(w) * scale), fh = std::floor(double(h) * scale);
  SPLAT_CHECK(fw <= double(1 << 30) && fh <= double(1 << 30), BAD_ARGUMENT,
              "image size: the cover of a " + std::to_string(w) + "x" + std::to_string(h) + " image is too large");
  rw = int(fw);
  rh = int(fh);
  left = (rw - width) / 2;
  top = (rh - height) / 2;
}

// --- host tables ---------------------------------------------------------------------------

namespace {

constexpr int TRAINED_GRID = 37;

std::array<double, 4> bicubic_weights(double t) {
  const double a = -0.75;
  auto near = [a](double x) { return ((a + 2.0) * x - (a + 3.0)) * x * x + 1.0; };
  auto far = [a](double x) { return ((a * x - 5.0 * a) * x + 8.0 * a) * x - 4.0 * a; };
  return {far(t + 1.0), near(t), near(1.0 - t), far(2.0 - t)};
}

struct Taps {
  int idx[4];
  double w[4];
};

std::vector<Taps> bicubic_taps(int in, int out, double scale) {
  std::vector<Taps> taps(out);
  for (int o = 0; o < out; ++o) {
    const double src = (o + 0.5) / scale - 0.5;
    const double fl = std::floor(src);
    auto w = bicubic_weights(src - fl);
    for (int i = 0; i < 4; ++i) {
      long v = long(fl) + i - 1;
      taps[o].idx[i] = int(std::min<long>(std::max<long>(v, 0), in - 1));
      taps[o].w[i] = w[i];
    }
  }
  return taps;
}

}  // namespace

// mapanything-rs/src/dinov2.rs:42-76 (separable bicubic, f64, columns then rows) applied as
// depthanything3-rs/src/backbone.rs:94-112: class slot kept, scale (out + 0.1) / 37.
std::vector<float> resize_pos_embed(const std::vector<float>& pos, int dim, int rows, int cols) {
  const int G = TRAINED_GRID;
  SPLAT_CHECK(dim > 0 && rows > 0 && cols > 0 && pos.size() >= size_t(1 + G * G) * dim, BAD_ARGUMENT,
              "positional embedding: sizes");
  std::vector<float> out(size_t(1 + rows * cols) * dim);
  std::memcpy(out.data(), pos.data(), sizeof(float) * dim);
  if (rows == G && cols == G) {
    std::memcpy(out.data(), pos.data(), sizeof(float) * out.size());
    return out;
  }
  const float* grid = pos.data() + dim;
  auto ct = bicubic_taps(G, cols, (cols + 0.1) / G);
  std::vector<double> horiz(size_t(G) * cols * dim, 0.0);
  for (int r = 0; r < G; ++r)
    for (int oc = 0; oc < cols; ++oc) {
      double* dst = &horiz[(size_t(r) * cols + oc) * dim];
      for (int t = 0; t < 4; ++t) {
        const float* src = grid + (size_t(r) * G + ct[oc].idx[t]) * dim;
        for (int c = 0; c < dim; ++c) dst[c] += ct[oc].w[t] * double(src[c]);
      }
    }
  auto rt = bicubic_taps(G, rows, (rows + 0.1) / G);
  for (int orow = 0; orow < rows; ++orow)
    for (int oc = 0; oc < cols; ++oc) {
      float* dst = &out[(1 + size_t(orow) * cols + oc) * dim];
      for (int c = 0; c < dim; ++c) {
        double s = 0.0;
        for (int t = 0; t < 4; ++t) s += rt[orow].w[t] * horiz[(size_t(rt[orow].idx[t]) * cols + oc) * dim + c];
        dst[c] = float(s);
      }
    }
  return out;
}

// depthanything3-rs/src/rope.rs:26-54: angle = pos * 100^(-p/16) in f64, stored f32.
std::vector<float> rope_table(int npos) {
  SPLAT_CHECK(npos >= 0, BAD_ARGUMENT, "rope table: positions");
  std::vector<float> t(size_t(2) * npos * 16);
  for (int pos = 0; pos < npos; ++pos)
    for (int p = 0; p < 16; ++p) {
      const double ang = double(pos) * (1.0 / std::pow(100.0, double(p) / 16.0));
      t[size_t(pos) * 16 + p] = float(std::cos(ang));
      t[size_t(npos) * 16 + size_t(pos) * 16 + p] = float(std::sin(ang));
    }
  return t;
}

// depthanything3-rs/src/uv_embed.rs:14-53, laid out [pixel][channel].
std::vector<float> uv_table(int channels, int rows, int cols, double aspect) {
  SPLAT_CHECK(channels > 0 && channels % 4 == 0 && rows > 0 && cols > 0, BAD_ARGUMENT, "uv table: sizes");
  const double diag = std::sqrt(aspect * aspect + 1.0);
  const double span[2] = {aspect / diag, 1.0 / diag};
  auto coord = [&](int i, int count, int axis) {
    const double edge = span[axis] * (count - 1.0) / count;
    return count == 1 ? -edge : -edge + 2.0 * edge * i / (count - 1.0);
  };
  const int half = channels / 2, q = half / 2;
  std::vector<float> t(size_t(rows) * cols * channels);
  for (int r = 0; r < rows; ++r)
    for (int c = 0; c < cols; ++c) {
      float* dst = &t[(size_t(r) * cols + c) * channels];
      const double pos[2] = {coord(c, cols, 0), coord(r, rows, 1)};
      for (int axis = 0; axis < 2; ++axis)
        for (int k = 0; k < q; ++k) {
          const double ang = pos[axis] / std::pow(100.0, double(k) / q);
          dst[axis * half + k] = float(std::sin(ang)) * 0.1f;
          dst[axis * half + q + k] = float(std::cos(ang)) * 0.1f;
        }
    }
  return t;
}

}  // namespace splat
