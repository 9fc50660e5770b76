// Shared device/host helpers for the splathip library (gfx950 / CDNA4 only).
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>
#include <cstddef>
#include <stdexcept>
#include <string>
#include <vector>

#include "errors.h"

namespace splat {

using bf16 = uint16_t;  // bfloat16 storage
struct f16 {            // IEEE binary16 storage (the reference's --precision f16)
  uint16_t bits;
};

// --- errors (errors.h: Status, Error, SPLAT_CHECK) ------------------------------------------

#define SPLAT_HIP(expr)                                                                   \
  do {                                                                                     \
    hipError_t e_ = (expr);                                                                \
    if (e_ != hipSuccess)                                                                  \
      throw ::splat::Error(::splat::HIP_ERROR, std::string(#expr) + ": " + hipGetErrorString(e_)); \
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

// --- f16 conversion -----------------------------------------------------------------------

__host__ __device__ inline float h2f(uint16_t h) {
#if defined(__HIP_DEVICE_COMPILE__)
  return float(__builtin_bit_cast(_Float16, h));
#else
  const uint32_t sign = uint32_t(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  uint32_t u;
  if (e == 0) {  // zero or subnormal: m * 2^-24
    float f = float(m) * 5.9604644775390625e-8f;
    __builtin_memcpy(&u, &f, 4);
    u |= sign;
  } else if (e == 31) {
    u = sign | 0x7f800000u | (m << 13);
  } else {
    u = sign | ((e + 112) << 23) | (m << 13);
  }
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
#endif
}

// Round to nearest even, overflow to infinity, NaN kept quiet; on the device v_cvt_f16_f32.
__host__ __device__ inline uint16_t f2h(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
#else
  uint32_t x;
  __builtin_memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u, mant = x & 0x7fffffu;
  const int exp = int((x >> 23) & 0xffu);
  if (exp == 0xff) return uint16_t(sign | 0x7c00u | (mant ? 0x200u | (mant >> 13) : 0u));
  const int e = exp - 127 + 15;
  if (e >= 31) return uint16_t(sign | 0x7c00u);
  if (e <= 0) {  // subnormal result (or zero)
    if (e < -10) return uint16_t(sign);
    const uint32_t m = mant | 0x800000u;
    const int shift = 14 - e;
    uint32_t h = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1u))) ++h;
    return uint16_t(sign | h);
  }
  uint32_t h = (uint32_t(e) << 10) | (mant >> 13);
  const uint32_t rem = mant & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;  // a carry into the exponent is right
  return uint16_t(sign | h);
#endif
}

typedef _Float16 f16x2_hw __attribute__((ext_vector_type(2)));
// Two floats -> packed f16 pair (low = a), rounded to nearest even.
__host__ __device__ inline uint32_t pack_f16x2(float a, float b) {
#if defined(__HIP_DEVICE_COMPILE__)
  f16x2_hw v = {static_cast<_Float16>(a), static_cast<_Float16>(b)};
  return __builtin_bit_cast(uint32_t, v);
#else
  return uint32_t(f2h(a)) | (uint32_t(f2h(b)) << 16);
#endif
}

template <typename T> __host__ __device__ inline float to_f(T v);
template <> __host__ __device__ inline float to_f<float>(float v) { return v; }
template <> __host__ __device__ inline float to_f<bf16>(bf16 v) { return bf2f(v); }
template <> __host__ __device__ inline float to_f<f16>(f16 v) { return h2f(v.bits); }

template <typename T> __host__ __device__ inline T from_f(float v);
template <> __host__ __device__ inline float from_f<float>(float v) { return v; }
template <> __host__ __device__ inline bf16 from_f<bf16>(float v) { return f2bf(v); }
template <> __host__ __device__ inline f16 from_f<f16>(float v) { return f16{f2h(v)}; }

// The 16-bit storage types (bf16, f16) by their raw bits: one value from the low 16 bits, and
// two floats packed (low = a).
template <typename T> __host__ __device__ inline float u16f(uint32_t bits);
template <> __host__ __device__ inline float u16f<bf16>(uint32_t bits) { return bf2f(bf16(bits & 0xffffu)); }
template <> __host__ __device__ inline float u16f<f16>(uint32_t bits) { return h2f(uint16_t(bits & 0xffffu)); }
template <typename T> __host__ __device__ inline uint32_t pack2(float a, float b);
template <> __host__ __device__ inline uint32_t pack2<bf16>(float a, float b) { return pack_bf16x2(a, b); }
template <> __host__ __device__ inline uint32_t pack2<f16>(float a, float b) { return pack_f16x2(a, b); }

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
__host__ __device__ inline int xcd_contiguous(int b, int nblk) {
  const int x = b & 7, q8 = nblk >> 3, r8 = nblk & 7;
  return (x < r8 ? x * (q8 + 1) : r8 * (q8 + 1) + (x - r8) * q8) + (b >> 3);
}
#endif

}  // namespace splat
