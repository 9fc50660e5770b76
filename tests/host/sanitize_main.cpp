// Host-only driver of the sanitizer test (tests/test_host_sanitize.py): the library's checkpoint
// parser (splatting-rs_amd/csrc/safetensors.cpp) and host tables (host_tables.cpp), built with a
// plain C++ compiler under AddressSanitizer and UndefinedBehaviorSanitizer. No GPU code.
//   sanitize_main parse <file>   parse the file through its memory map and through a byte copy,
//                                then convert every tensor to f32 with its own shape; prints
//                                "OK <tensors>" or "ERR <status> <message>" per path
//   sanitize_main tables         the per-grid tables, resize taps and size rules over ordinary
//                                and edge sizes; prints one line per case
#include <cmath>
#include <cstdio>
#include <fstream>
#include <functional>
#include <iterator>
#include <string>
#include <vector>

#include "../../splatting-rs_amd/csrc/host_tables.h"
#include "../../splatting-rs_amd/csrc/safetensors.h"

using namespace splat;

static void run(const std::string& label, const std::function<std::string()>& fn) {
  try {
    std::printf("%s OK %s\n", label.c_str(), fn().c_str());
  } catch (const Error& e) {
    std::printf("%s ERR %d %s\n", label.c_str(), e.code, e.what());
  }
}

static std::string convert_all(const SafeTensors& st) {
  double sum = 0.0;
  for (const auto& name : st.names()) {
    const StTensor& t = st.get(name);
    if (t.dtype != "F32" && t.dtype != "BF16" && t.dtype != "F16" && t.dtype != "F64") continue;
    for (float v : st.f32(name, t.shape)) sum += std::isfinite(v) ? v : 0.0;
  }
  return std::to_string(st.names().size()) + " " + std::to_string(sum);
}

static int parse(const char* path) {
  run("map", [&] {
    SafeTensors st;
    st.open_file(path);
    return convert_all(st);
  });
  run("bytes", [&] {
    std::ifstream f(path, std::ios::binary);
    std::vector<uint8_t> data((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
    SafeTensors st;
    st.open_bytes(data.data(), data.size());
    return convert_all(st);
  });
  return 0;
}

static std::string checksum(const std::vector<float>& v) {
  double s = 0.0;
  for (float x : v) s += x;
  return std::to_string(v.size()) + " " + std::to_string(s);
}

static int tables() {
  const int G = 37;
  for (int dim : {1, 64}) {
    std::vector<float> pos(size_t(1 + G * G) * dim);
    for (size_t i = 0; i < pos.size(); ++i) pos[i] = float(std::sin(0.37 * double(i)));
    for (auto rc : std::vector<std::pair<int, int>>{{1, 1}, {2, 3}, {27, 36}, {28, 37}, {37, 37}, {80, 80}})
      run("pos " + std::to_string(dim) + " " + std::to_string(rc.first) + "x" + std::to_string(rc.second),
          [&] { return checksum(resize_pos_embed(pos, dim, rc.first, rc.second)); });
    run("pos short", [&] { return checksum(resize_pos_embed(std::vector<float>(10), dim, 2, 2)); });
  }
  for (int n : {0, 1, 2000, -1}) run("rope " + std::to_string(n), [&] { return checksum(rope_table(n)); });
  for (auto c : std::vector<std::array<int, 3>>{{4, 1, 1}, {384, 27, 36}, {32, 504, 504}, {6, 2, 2}, {32, 0, 4}})
    run("uv " + std::to_string(c[0]) + " " + std::to_string(c[1]) + "x" + std::to_string(c[2]),
        [&] { return checksum(uv_table(c[0], c[1], c[2], double(c[2]) / double(c[1] ? c[1] : 1))); });
  for (int f = SPLAT_FILTER_TRIANGLE; f <= SPLAT_FILTER_LANCZOS3 + 1; ++f)
    for (auto io : std::vector<std::pair<int, int>>{{1, 1000}, {1000, 1}, {7, 7}, {1, 1}, {3, 2}, {4032, 518}, {0, 5}})
      run("taps " + std::to_string(f) + " " + std::to_string(io.first) + "->" + std::to_string(io.second), [&] {
        ResizeTapsHost t = resize_taps(io.first, io.second, f);
        double worst = 0.0;  // every output's weights sum to one; every tap lies inside the input
        for (size_t o = 0; o < t.first.size(); ++o) {
          double s = 0.0;
          for (int i = 0; i < t.count[o]; ++i) s += t.w[size_t(t.offset[o] + i)];
          worst = std::max(worst, std::fabs(s - 1.0));
          if (t.first[o] < 0 || t.count[o] < 1 || t.first[o] + t.count[o] > io.first) return std::string("tap out of range");
        }
        return std::to_string(t.w.size()) + " sum_dev " + std::to_string(worst);
      });
  for (auto wh : std::vector<std::pair<int, int>>{{1, 1}, {1, 1 << 30}, {504, 504}, {4032, 3024}, {0, 5}, {-3, 7}})
    run("da3_size " + std::to_string(wh.first) + "x" + std::to_string(wh.second), [&] {
      int bw, bh, w, h;
      da3_model_input_size(wh.first, wh.second, bw, bh, w, h);
      return std::to_string(bw) + " " + std::to_string(bh) + " " + std::to_string(w) + " " + std::to_string(h);
    });
  for (auto wh : std::vector<std::pair<int, int>>{{1000, 700}, {1, 1 << 30}, {1 << 30, 1}, {518, 392}, {0, 1}})
    run("ma_size " + std::to_string(wh.first) + "x" + std::to_string(wh.second), [&] {
      int W, H, rw, rh, left, top, filter;
      ma_input_size(1, &wh.first, &wh.second, W, H);
      ma_cover(wh.first, wh.second, W, H, rw, rh, left, top, filter);
      return std::to_string(W) + "x" + std::to_string(H) + " cover " + std::to_string(rw) + "x" + std::to_string(rh);
    });
  run("ma_size none", [&] {
    int W, H;
    ma_input_size(0, nullptr, nullptr, W, H);
    return std::string("?");
  });
  return 0;
}

int main(int argc, char** argv) {
  if (argc == 3 && std::string(argv[1]) == "parse") return parse(argv[2]);
  if (argc == 2 && std::string(argv[1]) == "tables") return tables();
  std::fprintf(stderr, "usage: %s parse <file> | tables\n", argv[0]);
  return 2;
}
