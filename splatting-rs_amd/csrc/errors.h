// Status codes and the error type of the library's host code, without HIP: shared by the
// runtime (common.h adds the HIP-call check) and by the host-only sources (the checkpoint
// parser, the host tables) that a plain C++ compiler builds for the sanitizer test.
#pragma once

#include <stdexcept>
#include <string>

namespace splat {

enum Status {
  OK = 0, BAD_ARGUMENT = 1, BAD_SHAPE = 2, MISSING_KEY = 3, SHAPE_MISMATCH = 4,
  HIP_ERROR = 5, NONFINITE = 6, IO_ERROR = 7, NOT_LOADED = 8
};

struct Error : std::runtime_error {
  int code;
  Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

}  // namespace splat

#define SPLAT_CHECK(cond, code, msg)                                                      \
  do {                                                                                     \
    if (!(cond)) throw ::splat::Error((code), (msg));                                     \
  } while (0)
