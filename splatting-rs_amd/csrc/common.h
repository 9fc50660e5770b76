// Shared device/host helpers for the splathip library (gfx950 / CDNA4 only).
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>
#include <cstddef>
#include <stdexcept>
#include <string>
#include <vector>

namespace splat {

using bf16 = uint16_t;  // bfloat16 storage

// --- errors -------------------------------------------------------------------------------

enum Status {
  OK = 0, BAD_ARGUMENT = 1, BAD_SHAPE = 2, MISSING_KEY = 3, SHAPE_MISMATCH = 4,
  HIP_ERROR = 5, NONFINITE = 6, IO_ERROR = 7, NOT_LOADED = 8
};

struct Error : std::runtime_error {
  int code;
  Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

#define SPLAT_HIP(expr)                                                                   \
  do {                                                                                     \
    hipError_t e_ = (expr);                                                                \
    if (e_ != hipSuccess)                                                                  \
      throw ::splat::Error(::splat::HIP_ERROR, std::string(#expr) + ": " + hipGetErrorString(e_)); \
  } while (0)

#define SPLAT_CHECK(cond, code, msg)                                                      \
  do {                                                                                     \
    if (!(cond)) throw ::splat::Error((code), (msg));                                     \
  } while (0)

// --- bf16 conversion ----------------------------------------------------------------------

__host__ __device__ inline float bf2f(bf16 v) {
  uint32_t u = uint32_t(v) << 16;
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}

// Round to nearest even (NaN kept quiet); on the device the v_cvt_pk_bf16_f32 instruction.
__host__ __device__ inline bf16 f2bf(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_bit_cast(bf16, static_cast<__bf16>(f));
#else
  uint32_t u;
  __builtin_memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return bf16((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return bf16(u >> 16);
#endif
}

typedef __bf16 bf16x2_hw __attribute__((ext_vector_type(2)));
// Two floats -> packed bf16 pair (low = a); on the device one v_cvt_pk_bf16_f32.
__host__ __device__ inline uint32_t pack_bf16x2(float a, float b) {
#if defined(__HIP_DEVICE_COMPILE__)
  bf16x2_hw v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(uint32_t, v);
#else
  return uint32_t(f2bf(a)) | (uint32_t(f2bf(b)) << 16);
#endif
}

template <typename T> __host__ __device__ inline float to_f(T v);
template <> __host__ __device__ inline float to_f<float>(float v) { return v; }
template <> __host__ __device__ inline float to_f<bf16>(bf16 v) { return bf2f(v); }

template <typename T> __host__ __device__ inline T from_f(float v);
template <> __host__ __device__ inline float from_f<float>(float v) { return v; }
template <> __host__ __device__ inline bf16 from_f<bf16>(float v) { return f2bf(v); }

// --- execution context for launches -------------------------------------------------------

// Per-launch timing records: HIP events around each launch on the launch's own stream, with
// the launch's algorithmic work (2*MAC flops, bytes of inputs read once + outputs written once).
struct ProfRecord {
  const char* name;
  double flops, bytes;
  hipEvent_t e0, e1;
};
struct Profiler {
  std::vector<ProfRecord> recs;
};

// Device scratch for split-K partial sums, owned by the context and shared by the launches
// of its stream (one at a time). A dry run records in `need` the bytes the real run will ask
// for; a launch splits only when `cap` covers its partials.
struct Workspace {
  void* ptr = nullptr;
  size_t cap = 0, need = 0;
};

// Every launcher receives an Exec. With `dry` set, launchers only validate their arguments
// and return: the forward runs once that way to size the activation arena (and `ws`).
struct Exec {
  hipStream_t stream = nullptr;
  bool dry = false;
  Profiler* prof = nullptr;
  Workspace* ws = nullptr;
};

// Records one launch when profiling: construct right before the launch, destroyed after it.
struct ProfScope {
  const Exec& ex;
  ProfRecord rec{};
  bool on;
  ProfScope(const Exec& e, const char* name, double flops, double bytes) : ex(e), on(e.prof != nullptr && !e.dry) {
    if (!on) return;
    rec.name = name;
    rec.flops = flops;
    rec.bytes = bytes;
    (void)hipEventCreate(&rec.e0);
    (void)hipEventCreate(&rec.e1);
    (void)hipEventRecord(rec.e0, ex.stream);
  }
  ~ProfScope() {
    if (!on) return;
    (void)hipEventRecord(rec.e1, ex.stream);
    ex.prof->recs.push_back(rec);
  }
};

inline int cdiv(long a, long b) { return int((a + b - 1) / b); }

#ifdef __HIPCC__
// Work-item order for a 1D grid of nblk workgroups: the dispatcher deals workgroups b, b+8,
// b+16, ... to one of the 8 XCDs (each with its own L2), so XCD x gets the contiguous range of
// logical ids starting at x*(nblk/8) (the first nblk%8 XCDs one id more). Neighbouring ids
// then share operands in one L2. A bijection of [0, nblk).
__device__ inline int xcd_contiguous(int b, int nblk) {
  const int x = b & 7, q8 = nblk >> 3, r8 = nblk & 7;
  return (x < r8 ? x * (q8 + 1) : r8 * (q8 + 1) + (x - r8) * q8) + (b >> 3);
}
#endif

}  // namespace splat
