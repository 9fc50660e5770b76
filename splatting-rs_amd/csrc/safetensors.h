// Minimal safetensors reader: 8-byte little-endian header length, a JSON header mapping
// tensor names to {dtype, shape, data_offsets}, then the raw little-endian data. Files are
// memory-mapped (the reference maps them too: depthanything3-rs/src/weights.rs:40-41);
// byte buffers are borrowed or copied (weights.rs:51-60).
#pragma once

#include <cstdint>
#include <map>
#include <string>
#include <vector>

namespace splat {

struct StTensor {
  std::string dtype;           // "F32", "BF16", "F16", ...
  std::vector<int64_t> shape;
  const uint8_t* data = nullptr;
  size_t nbytes = 0;
  // Parsed shapes are checked (no negative dimension, byte size within int64_t), so this
  // product does not overflow.
  int64_t numel() const {
    int64_t n = 1;
    for (auto s : shape) n *= s;
    return n;
  }
};

class SafeTensors {
 public:
  SafeTensors() = default;
  SafeTensors(const SafeTensors&) = delete;
  SafeTensors& operator=(const SafeTensors&) = delete;
  ~SafeTensors();

  void open_file(const std::string& path);
  void open_bytes(const uint8_t* bytes, size_t len);   // copies the bytes

  bool has(const std::string& name) const { return tensors_.count(name) != 0; }
  std::vector<std::string> names() const {
    std::vector<std::string> r;
    for (const auto& kv : tensors_) r.push_back(kv.first);
    return r;
  }
  const StTensor& get(const std::string& name) const;  // throws MISSING_KEY
  // The tensor converted to f32, after checking its shape (throws SHAPE_MISMATCH).
  std::vector<float> f32(const std::string& name, const std::vector<int64_t>& shape) const;

 private:
  void parse(const uint8_t* base, size_t len);
  void* map_ = nullptr;
  size_t map_len_ = 0;
  std::vector<uint8_t> owned_;
  std::map<std::string, StTensor> tensors_;
};

std::string shape_str(const std::vector<int64_t>& s);

}  // namespace splat
