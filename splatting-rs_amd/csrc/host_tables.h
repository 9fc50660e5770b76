// Host-side tables and size rules (host_tables.cpp), declared without HIP.
#pragma once

#include <vector>

#include "../../include/splathip.h"
#include "errors.h"

namespace splat {

// --- image preprocessing -----------------------------------------------------------------------

// Host taps of one resize axis (image 0.25.10 sample.rs): output o reads count[o] inputs from
// first[o] with the normalised weights w[offset[o] ..].
struct ResizeTapsHost {
  std::vector<int> first, count, offset;
  std::vector<float> w;
};
ResizeTapsHost resize_taps(int in, int out, int filter);
void da3_model_input_size(int width, int height, int& bw, int& bh, int& dw, int& dh);
int da3_resize_filter(int w, int h, int nw, int nh);
void ma_input_size(int n, const int* widths, const int* heights, int& width, int& height);
void ma_cover(int w, int h, int width, int height, int& rw, int& rh, int& left, int& top, int& filter);

// --- per-grid tables (f64 on the host, stored f32) ----------------------------------------------

std::vector<float> resize_pos_embed(const std::vector<float>& pos, int dim, int rows, int cols);  // [1+P, d]
std::vector<float> rope_table(int npos);                                                        // [2][npos][16]
std::vector<float> uv_table(int channels, int rows, int cols, double aspect);                   // [rows*cols, C]

}  // namespace splat
