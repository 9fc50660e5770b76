// HBM-bound and small kernels around the GEMMs and attention: LayerNorms, row statistics,
// patch im2col, bilinear resize (align_corners=True), DPT output heads, small head linears,
// DA3 reference-view selection and hook assembly, and elementwise helpers.
#include "kernels.h"

#include <algorithm>

namespace splat {

namespace {

template <typename T> __device__ inline float ld(const void* p, long i) { return to_f<T>(reinterpret_cast<const T*>(p)[i]); }
template <typename T> __device__ inline void st(void* p, long i, float v) { reinterpret_cast<T*>(p)[i] = from_f<T>(v); }

// v + the value of lane l' for the DPP lane pattern CTRL (the pairing of a reduction step).
template <int CTRL> __device__ inline float dpp_add(float v) {
  const int o = __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, true);
  return v + __int_as_float(o);
}

// Sum over the wave, left in every lane, without LDS: DPP within each 16-lane row (quad swaps,
// half-row mirror, row mirror), then v_permlane16_swap (lane l and l ^ 16 exchange) and
// v_permlane32_swap (l and l ^ 32).
__device__ inline float wave_sum(float v) {
  v = dpp_add<0xB1>(v);   // quad_perm [1,0,3,2]
  v = dpp_add<0x4E>(v);   // quad_perm [2,3,0,1]
  v = dpp_add<0x141>(v);  // row_half_mirror
  v = dpp_add<0x140>(v);  // row_mirror
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
__device__ inline double wave_sum_d(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

inline int in_dt_ok(int dt) { return dt == F32 || dt == BF16 || dt == F16; }

// Calls f with a value of Ty<T> for the element type T of dtype dt (float, bf16 or f16).
template <typename T> struct Ty { using type = T; };
template <typename F> inline void by_dt(int dt, F&& f) {
  if (dt == F32) f(Ty<float>{});
  else if (dt == F16) f(Ty<f16>{});
  else f(Ty<bf16>{});
}
#define TY(t) typename decltype(t)::type

}  // namespace

// ---------------------------------------------------------------------------------------
// LayerNorm over rows, one wave per row, two passes (mean, then centred variance) with the
// row re-read from cache. Biased variance and eps inside the sqrt, as torch/candle.
template <typename TI, typename TO>
__global__ void ln_kernel(const void* in, long ldin, void* out, long ldout, int rows, int n, const float* w,
                          const float* b, float eps, int rmP, int rmn, int rmoff) {
  const int wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6, lane = threadIdx.x & 63;
  if (wave >= rows) return;
  const long rin = rmP ? (long)(wave / rmP) * rmn + rmoff + wave % rmP : wave;
  const long ib = rin * ldin, ob = (long)wave * ldout;
  float s = 0.f;
  for (int c = lane; c < n; c += 64) s += ld<TI>(in, ib + c);
  const float mean = wave_sum(s) / n;
  float v = 0.f;
  for (int c = lane; c < n; c += 64) {
    const float d = ld<TI>(in, ib + c) - mean;
    v += d * d;
  }
  const float rstd = rsqrtf(wave_sum(v) / n + eps);
  for (int c = lane; c < n; c += 64) {
    float y = (ld<TI>(in, ib + c) - mean) * rstd;
    if (w) y = y * w[c] + b[c];
    st<TO>(out, ob + c, y);
  }
}

// 4 consecutive elements as floats / from floats (16-byte fp32 or 8-byte bf16/f16 accesses).
template <typename T> __device__ inline float4 ld4(const void* p, long i) {
  if constexpr (sizeof(T) == 4) {
    return *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(p) + i);
  } else {
    const uint2 u = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(p) + i);
    return make_float4(u16f<T>(u.x), u16f<T>(u.x >> 16), u16f<T>(u.y), u16f<T>(u.y >> 16));
  }
}
template <typename T> __device__ inline void st4(void* p, long i, float4 v) {
  if constexpr (sizeof(T) == 4)
    *reinterpret_cast<float4*>(reinterpret_cast<float*>(p) + i) = v;
  else
    *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(p) + i) = make_uint2(pack2<T>(v.x, v.y), pack2<T>(v.z, v.w));
}

// Register-resident LayerNorm: one wave per row, 4-element vector accesses, the row held in
// MAXC float4 per lane; mean, then centred variance, from registers.
template <typename TI, typename TO, int MAXC>
__global__ void ln_vec_kernel(const void* in, long ldin, void* out, long ldout, int rows, int n, const float* w,
                              const float* b, float eps, int rmP, int rmn, int rmoff) {
  const int wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6, lane = threadIdx.x & 63;
  if (wave >= rows) return;
  const long rin = rmP ? (long)(wave / rmP) * rmn + rmoff + wave % rmP : wave;
  const long ib = rin * ldin, ob = (long)wave * ldout;
  const int nc = n >> 2;
  float4 x[MAXC];
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < MAXC; ++k) {
    const int c = lane + 64 * k;
    x[k] = c < nc ? ld4<TI>(in, ib + 4 * c) : make_float4(0.f, 0.f, 0.f, 0.f);
    s += (x[k].x + x[k].y) + (x[k].z + x[k].w);
  }
  const float mean = wave_sum(s) / n;
  float q = 0.f;
#pragma unroll
  for (int k = 0; k < MAXC; ++k) {
    if (lane + 64 * k < nc) {
      const float a = x[k].x - mean, bb = x[k].y - mean, cc = x[k].z - mean, d = x[k].w - mean;
      q += (a * a + bb * bb) + (cc * cc + d * d);
    }
  }
  const float rstd = rsqrtf(wave_sum(q) / n + eps);
#pragma unroll
  for (int k = 0; k < MAXC; ++k) {
    const int c = lane + 64 * k;
    if (c < nc) {
      float4 y = make_float4((x[k].x - mean) * rstd, (x[k].y - mean) * rstd, (x[k].z - mean) * rstd, (x[k].w - mean) * rstd);
      if (w) {
        const float4 wv = *reinterpret_cast<const float4*>(w + 4 * c), bv = *reinterpret_cast<const float4*>(b + 4 * c);
        y = make_float4(y.x * wv.x + bv.x, y.y * wv.y + bv.y, y.z * wv.z + bv.z, y.w * wv.w + bv.w);
      }
      st4<TO>(out, ob + 4 * c, y);
    }
  }
}

template <typename TI, typename TO>
static void ln_launch(const Exec& ex, const void* in, long ldin, void* out, long ldout, int rows, int n, const float* w,
                      const float* b, float eps, int rm_P, int rm_n, int rm_off) {
  dim3 grid(cdiv(rows, 4));
  const int per_lane = cdiv(n / 4, 64);
  const bool vec = n % 4 == 0 && ldin % 4 == 0 && ldout % 4 == 0 && per_lane <= 16 &&
                   (reinterpret_cast<uintptr_t>(in) & 15) == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0;
  if (!vec) {
    hipLaunchKernelGGL((ln_kernel<TI, TO>), grid, dim3(256), 0, ex.stream, in, ldin, out, ldout, rows, n, w, b, eps, rm_P, rm_n, rm_off);
  } else if (per_lane <= 2) {
    hipLaunchKernelGGL((ln_vec_kernel<TI, TO, 2>), grid, dim3(256), 0, ex.stream, in, ldin, out, ldout, rows, n, w, b, eps, rm_P, rm_n, rm_off);
  } else if (per_lane <= 4) {
    hipLaunchKernelGGL((ln_vec_kernel<TI, TO, 4>), grid, dim3(256), 0, ex.stream, in, ldin, out, ldout, rows, n, w, b, eps, rm_P, rm_n, rm_off);
  } else if (per_lane <= 8) {
    hipLaunchKernelGGL((ln_vec_kernel<TI, TO, 8>), grid, dim3(256), 0, ex.stream, in, ldin, out, ldout, rows, n, w, b, eps, rm_P, rm_n, rm_off);
  } else {
    hipLaunchKernelGGL((ln_vec_kernel<TI, TO, 16>), grid, dim3(256), 0, ex.stream, in, ldin, out, ldout, rows, n, w, b, eps, rm_P, rm_n, rm_off);
  }
}

void layer_norm(const Exec& ex, int in_dt, const void* in, long ldin, int out_dt, void* out, long ldout, int rows,
                int n, const float* w, const float* b, float eps, int rm_P, int rm_n, int rm_off) {
  SPLAT_CHECK(in_dt_ok(in_dt) && in_dt_ok(out_dt) && rows >= 0 && n > 0, BAD_ARGUMENT, "layer_norm args");
  SPLAT_CHECK((w == nullptr) == (b == nullptr), BAD_ARGUMENT, "layer_norm: weight and bias come together");
  if (ex.dry || rows == 0) return;
  ProfScope ps(ex, "layer_norm", 0, double(rows) * n * (dtype_size(in_dt) + dtype_size(out_dt)));
  by_dt(in_dt, [&](auto ti) {
    by_dt(out_dt, [&](auto to) { ln_launch<TY(ti), TY(to)>(ex, in, ldin, out, ldout, rows, n, w, b, eps, rm_P, rm_n, rm_off); });
  });
  SPLAT_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------------------
// Row statistics for a LayerNorm folded into the next GEMM (GemmArgs::ln_in): one wave per
// row, 4 columns a lane; the 16 lanes of a DPP row cover 64 columns, so each 64-column sum is a
// 16-lane reduction (a 128-column group adds two of them); optional copy of the row in the
// GEMM's dtype.
template <typename TO>
__global__ void __launch_bounds__(256) ln_stats_kernel(const float* x, long ldx, int rows, int n, int group,
                                                       float* stats, void* copy, int rmP, int rmn, int rmoff) {
  const int wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6, lane = threadIdx.x & 63;
  if (wave >= rows) return;  // whole waves leave together
  const long row = rmP ? (long)(wave / rmP) * rmn + rmoff + wave % rmP : wave;
  const int nc = n >> 2, parts = n / group;
  for (int k = 0; k * 64 < nc; ++k) {
    const int c = lane + 64 * k;
    float s = 0.f, q = 0.f;
    if (c < nc) {
      const float4 v = ld4<float>(x, row * ldx + 4 * c);
      s = (v.x + v.y) + (v.z + v.w);
      q = (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
      if (copy) st4<TO>(copy, row * ldx + 4 * c, v);
    }
    s = dpp_add<0x140>(dpp_add<0x141>(dpp_add<0x4E>(dpp_add<0xB1>(s))));  // over the 16 lanes
    q = dpp_add<0x140>(dpp_add<0x141>(dpp_add<0x4E>(dpp_add<0xB1>(q))));
    if (group == 128) {  // lanes l and l ^ 16 hold the two halves of a 128-column group
      s += __shfl_xor(s, 16);
      q += __shfl_xor(q, 16);
    }
    const int g = (4 * c) / group;
    if ((lane & (group / 4 - 1)) == 0 && c < nc) {
      stats[(row * parts + g) * 2] = s;
      stats[(row * parts + g) * 2 + 1] = q;
    }
  }
}

void ln_stats(const Exec& ex, const float* x, long ldx, int rows, int n, int group, float* stats, int copy_dt,
              void* copy, int rm_P, int rm_n, int rm_off) {
  SPLAT_CHECK(rows >= 0 && (group == 64 || group == 128) && n % group == 0 && ldx % 4 == 0 && in_dt_ok(copy_dt),
              BAD_ARGUMENT, "ln_stats args");
  SPLAT_CHECK((reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(copy) & 15) == 0, BAD_ARGUMENT,
              "ln_stats: 16-byte aligned rows");
  if (ex.dry || rows == 0) return;
  ProfScope ps(ex, "ln_stats", 0, double(rows) * n * (4 + (copy ? dtype_size(copy_dt) : 0)));
  dim3 grid(cdiv(rows, 4));
  by_dt(copy_dt, [&](auto t) {
    hipLaunchKernelGGL(ln_stats_kernel<TY(t)>, grid, dim3(256), 0, ex.stream, x, ldx, rows, n, group, stats, copy, rm_P, rm_n, rm_off);
  });
  SPLAT_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------------------
template <typename T>
__global__ void im2col_kernel(const float* img, int V, int H, int W, void* out, int kpad) {
  const int R = H / 14, C = W / 14;
  const long id = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long total = (long)V * R * C * kpad;
  if (id >= total) return;
  const int k = int(id % kpad);
  const long pidx = id / kpad;
  float v = 0.f;
  if (k < 588) {
    const int c = k / 196, rem = k % 196, ky = rem / 14, kx = rem % 14;
    const long vv = pidx / (R * C);
    const int pp = int(pidx % (R * C)), py = pp / C, px = pp % C;
    v = img[((vv * 3 + c) * H + py * 14 + ky) * W + px * 14 + kx];
  }
  st<T>(out, id, v);
}

void im2col_patch(const Exec& ex, int dt, const float* img, int V, int H, int W, void* out, int kpad) {
  SPLAT_CHECK(H % 14 == 0 && W % 14 == 0 && kpad >= 588, BAD_ARGUMENT, "im2col args");
  if (ex.dry) return;
  const long total = (long)V * (H / 14) * (W / 14) * kpad;
  ProfScope ps(ex, "im2col_patch", 0, double(V) * 3 * H * W * 4 + double(total) * dtype_size(dt));
  dim3 grid(cdiv(total, 256));
  by_dt(dt, [&](auto t) { hipLaunchKernelGGL(im2col_kernel<TY(t)>, grid, dim3(256), 0, ex.stream, img, V, H, W, out, kpad); });
  SPLAT_HIP(hipGetLastError());
}

__global__ void class_rows_kernel(float* xs, int V, int n, int dim, const float* cls, const float* pos0) {
  const long id = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= (long)V * dim) return;
  const int v = int(id / dim), c = int(id % dim);
  xs[(long)v * n * dim + c] = cls[c] + (pos0 ? pos0[c] : 0.f);
}

void write_class_rows(const Exec& ex, float* xs, int V, int n, int dim, const float* cls, const float* pos0) {
  if (ex.dry) return;
  hipLaunchKernelGGL(class_rows_kernel, dim3(cdiv((long)V * dim, 256)), dim3(256), 0, ex.stream, xs, V, n, dim, cls, pos0);
  SPLAT_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------------------
// Bilinear resize, align_corners=True (torch upsample_bilinear2d semantics: source =
// dst * (in-1)/(out-1) in fp32, lambdas from the fractional part), NHWC.
template <typename T>
__global__ void resize_kernel(const void* in, int V, int Hi, int Wi, int C, void* out, int Hf, int Wf, int Ho, int Wo,
                              const float* addtab, int relu) {
  const long id = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long total = (long)V * Ho * Wo * C;
  if (id >= total) return;
  const int c = int(id % C);
  long r = id / C;
  const int ox = int(r % Wo);
  r /= Wo;
  const int oy = int(r % Ho);
  const long v = r / Ho;
  // Source coordinates in f64 (exact to well below an fp32 ulp), weights in fp32.
  const double fy = Hf > 1 ? double(Hi - 1) * oy / double(Hf - 1) : 0.0;
  const double fx = Wf > 1 ? double(Wi - 1) * ox / double(Wf - 1) : 0.0;
  const int y0 = min(int(fy), Hi - 1), x0 = min(int(fx), Wi - 1);
  const int y1 = y0 + (y0 < Hi - 1 ? 1 : 0), x1 = x0 + (x0 < Wi - 1 ? 1 : 0);
  const float ly = float(fy - y0), lx = float(fx - x0);
  const long b = v * Hi * Wi;
  const float a00 = ld<T>(in, ((b + (long)y0 * Wi + x0) * C) + c);
  const float a01 = ld<T>(in, ((b + (long)y0 * Wi + x1) * C) + c);
  const float a10 = ld<T>(in, ((b + (long)y1 * Wi + x0) * C) + c);
  const float a11 = ld<T>(in, ((b + (long)y1 * Wi + x1) * C) + c);
  float val = (1.f - ly) * ((1.f - lx) * a00 + lx * a01) + ly * ((1.f - lx) * a10 + lx * a11);
  if (addtab) val += addtab[((long)oy * Wo + ox) * C + c];
  if (relu) val = fmaxf(val, 0.f);
  st<T>(out, id, val);
}

// Same, 8 channels per thread (C % 8 == 0): the four source pixels and the output are read
// and written as 8-channel vectors (one 16-byte access per pixel for bf16 and f16). One block row per
// output row (grid.y = V*Ho), so the row's source rows and weight follow from blockIdx.y and the
// per-thread index math is 32-bit (C4's five resizes 295 -> 230 us against a flat 64-bit index
// decomposition with 8-byte accesses). A thread covers RESIZE_ROWS output rows of one column, so
// the column's source coordinate is computed once; coordinates are f64 products with the scale
// (in - 1) / (out - 1) computed on the host (the f64 division per thread and row was most of
// the kernel's instructions).
template <typename T> struct Vec8 {  // the 16-bit types
  __device__ static inline void load(const void* p, long i, float* v) {
    const uint4 u = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(p) + i);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[2 * k] = u16f<T>(w[k]);
      v[2 * k + 1] = u16f<T>(w[k] >> 16);
    }
  }
  __device__ static inline void store(void* p, long i, const float* v) {
    uint4 u;
    u.x = pack2<T>(v[0], v[1]);
    u.y = pack2<T>(v[2], v[3]);
    u.z = pack2<T>(v[4], v[5]);
    u.w = pack2<T>(v[6], v[7]);
    *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(p) + i) = u;
  }
};
template <> struct Vec8<float> {
  __device__ static inline void load(const void* p, long i, float* v) {
    const float4 a = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(p) + i);
    const float4 b = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(p) + i + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
  __device__ static inline void store(void* p, long i, const float* v) {
    float* o = reinterpret_cast<float*>(p) + i;
    *reinterpret_cast<float4*>(o) = make_float4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<float4*>(o + 4) = make_float4(v[4], v[5], v[6], v[7]);
  }
};

constexpr int RESIZE_ROWS = 4;
template <typename T>
__global__ void __launch_bounds__(256) resize8_kernel(const void* in, int Hi, int Wi, int C, void* out, int Ho, int Wo,
                                                      int rows, double sy, double sx, const float* addtab, int relu) {
  const int C8 = C >> 3;
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= Wo * C8) return;
  const int ox = t / C8, c = (t - ox * C8) * 8;
  const double fx = sx * ox;
  const int x0 = min(int(fx), Wi - 1);
  const int x1 = x0 + (x0 < Wi - 1 ? 1 : 0);
  const float lx = float(fx - x0);
  for (int r = 0; r < RESIZE_ROWS; ++r) {
    const int row = blockIdx.y * RESIZE_ROWS + r;  // over V * Ho output rows
    if (row >= rows) break;
    const int v = row / Ho, oy = row - v * Ho;
    const double fy = sy * oy;
    const int y0 = min(int(fy), Hi - 1);
    const int y1 = y0 + (y0 < Hi - 1 ? 1 : 0);
    const float ly = float(fy - y0);
    const long b = long(v) * Hi * Wi;
    float a[8], bq[8], cq[8], d[8], y[8];
    Vec8<T>::load(in, (b + long(y0) * Wi + x0) * C + c, a);
    Vec8<T>::load(in, (b + long(y0) * Wi + x1) * C + c, bq);
    Vec8<T>::load(in, (b + long(y1) * Wi + x0) * C + c, cq);
    Vec8<T>::load(in, (b + long(y1) * Wi + x1) * C + c, d);
#pragma unroll
    for (int k = 0; k < 8; ++k) y[k] = (1.f - ly) * ((1.f - lx) * a[k] + lx * bq[k]) + ly * ((1.f - lx) * cq[k] + lx * d[k]);
    if (addtab) {
      const float* tp = addtab + (long(oy) * Wo + ox) * C + c;
      const float4 t0 = *reinterpret_cast<const float4*>(tp), t1 = *reinterpret_cast<const float4*>(tp + 4);
      y[0] += t0.x; y[1] += t0.y; y[2] += t0.z; y[3] += t0.w; y[4] += t1.x; y[5] += t1.y; y[6] += t1.z; y[7] += t1.w;
    }
    if (relu) {
#pragma unroll
      for (int k = 0; k < 8; ++k) y[k] = fmaxf(y[k], 0.f);
    }
    Vec8<T>::store(out, (long(row) * Wo + ox) * C + c, y);
  }
}

void resize_bilinear(const Exec& ex, int dt, const void* in, int V, int Hi, int Wi, int C, void* out, int Hf, int Wf,
                     int Ho, int Wo, const float* addtab, int relu) {
  SPLAT_CHECK(Ho <= Hf && Wo <= Wf && Hi > 0 && Wi > 0, BAD_ARGUMENT, "resize args");
  if (ex.dry) return;
  const long total = (long)V * Ho * Wo * C;
  if (C % 8 == 0 && (reinterpret_cast<uintptr_t>(in) & 15) == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0 &&
      (reinterpret_cast<uintptr_t>(addtab) & 15) == 0) {
    ProfScope ps(ex, "resize_bilinear", 0, (double(V) * Hi * Wi * C + double(total)) * dtype_size(dt) + (addtab ? double(Ho) * Wo * C * 4 : 0));
    const int rows = V * Ho;
    SPLAT_CHECK(long(Wo) * (C / 8) < (1L << 31) && cdiv(rows, RESIZE_ROWS) < 65536, BAD_ARGUMENT, "resize: grid");
    const double sy = Hf > 1 ? double(Hi - 1) / double(Hf - 1) : 0.0, sx = Wf > 1 ? double(Wi - 1) / double(Wf - 1) : 0.0;
    dim3 grid(cdiv(long(Wo) * (C / 8), 256), cdiv(rows, RESIZE_ROWS));
    by_dt(dt, [&](auto t) {
      hipLaunchKernelGGL(resize8_kernel<TY(t)>, grid, dim3(256), 0, ex.stream, in, Hi, Wi, C, out, Ho, Wo, rows, sy, sx, addtab, relu);
    });
    SPLAT_HIP(hipGetLastError());
    return;
  }
  ProfScope ps(ex, "resize_bilinear", 0, (double(V) * Hi * Wi * C + double(total)) * dtype_size(dt) + (addtab ? double(Ho) * Wo * C * 4 : 0));
  dim3 grid(cdiv(total, 256));
  by_dt(dt, [&](auto t) {
    hipLaunchKernelGGL(resize_kernel<TY(t)>, grid, dim3(256), 0, ex.stream, in, V, Hi, Wi, C, out, Hf, Wf, Ho, Wo, addtab, relu);
  });
  SPLAT_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------------------
// Output heads: one thread per pixel; weights (cout x cin fp32) staged in LDS.
template <typename T>
__global__ void pw_kernel(int mode, const void* in, long pix, int hw, int cin, int cout, const float* w, const float* b,
                          float* o0, float* o1, float* o2, uint8_t* o3, const float* scale) {
  __shared__ float sw[8 * 256];
  __shared__ float sb[8];
  for (int i = threadIdx.x; i < cout * cin; i += blockDim.x) sw[i] = w[i];
  if (threadIdx.x < cout) sb[threadIdx.x] = b[threadIdx.x];
  __syncthreads();
  const long px = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (px >= pix) return;
  const long base = px * cin;
  float mean = 0.f, rstd = 1.f;
  if (mode == PW_RAY) {
    float s = 0.f;
    for (int c = 0; c < cin; ++c) s += ld<T>(in, base + c);
    mean = s / cin;
    float q = 0.f;
    for (int c = 0; c < cin; ++c) {
      const float d = ld<T>(in, base + c) - mean;
      q += d * d;
    }
    rstd = rsqrtf(q / cin + 1e-5f);
  }
  float acc[8];
#pragma unroll
  for (int o = 0; o < 8; ++o) acc[o] = o < cout ? sb[o] : 0.f;
  for (int c = 0; c < cin; ++c) {
    float x = ld<T>(in, base + c);
    if (mode == PW_RAY) x = fmaxf((x - mean) * rstd, 0.f);
#pragma unroll
    for (int o = 0; o < 8; ++o)
      if (o < cout) acc[o] += sw[o * cin + c] * x;
  }
  const long v = px / hw, q = px % hw;
  if (mode == PW_DEPTH) {
    o0[px] = expf(acc[0]);
    o1[px] = 1.f + expf(acc[1]);
  } else if (mode == PW_RAY) {
    for (int o = 0; o < cout; ++o) o0[(v * cout + o) * hw + q] = acc[o];
  } else {
    if (o0)
      for (int o = 0; o < cout; ++o) o0[(v * cout + o) * hw + q] = acc[o];
    // mapanything-rs/src/model.rs:155-168
    const float nrm = fmaxf(sqrtf(acc[0] * acc[0] + acc[1] * acc[1] + acc[2] * acc[2]), 1e-8f);
    const float depth = expf(acc[3]) * (scale ? *scale : 1.f);
    if (o1) {
      o1[px * 3 + 0] = acc[0] / nrm * depth;
      o1[px * 3 + 1] = acc[1] / nrm * depth;
      o1[px * 3 + 2] = acc[2] / nrm * depth;
    }
    if (o2) o2[px] = 1.f + expf(acc[4]);
    if (o3) o3[px] = acc[5] > 0.f ? 1 : 0;
  }
}

// Cooperative form: LPP lanes per pixel (cin = 8*LPP), each lane holding 8 channels read as
// one vector; dot products and LayerNorm statistics are reduced across the lane group.
template <typename T, int LPP>
__global__ void pw_coop_kernel(int mode, const void* in, long pix, int hw, int cin, int cout, const float* w,
                               const float* b, float* o0, float* o1, float* o2, uint8_t* o3, const float* scale) {
  __shared__ float sw[8 * 256];
  __shared__ float sb[8];
  for (int i = threadIdx.x; i < cout * cin; i += blockDim.x) sw[i] = w[i];
  if (threadIdx.x < cout) sb[threadIdx.x] = b[threadIdx.x];
  __syncthreads();
  const long gt = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long px = gt / LPP;
  const int sub = int(gt % LPP);
  if (px >= pix) return;  // whole lane groups leave together (LPP divides 64)
  const int c0 = sub * 8;
  float x[8];
  {
    const float4 a = ld4<T>(in, px * cin + c0), bb = ld4<T>(in, px * cin + c0 + 4);
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = bb.x; x[5] = bb.y; x[6] = bb.z; x[7] = bb.w;
  }
  auto group_sum = [](float v) {
#pragma unroll
    for (int o = LPP / 2; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
  };
  if (mode == PW_RAY) {
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) s += x[k];
    const float mean = group_sum(s) / cin;
    float q = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) q += (x[k] - mean) * (x[k] - mean);
    const float rstd = rsqrtf(group_sum(q) / cin + 1e-5f);
#pragma unroll
    for (int k = 0; k < 8; ++k) x[k] = fmaxf((x[k] - mean) * rstd, 0.f);
  }
  float acc[8];
#pragma unroll
  for (int o = 0; o < 8; ++o) {
    float s = 0.f;
    if (o < cout) {
#pragma unroll
      for (int k = 0; k < 8; ++k) s += sw[o * cin + c0 + k] * x[k];
    }
    acc[o] = group_sum(s) + (o < cout ? sb[o] : 0.f);
  }
  if (sub != 0) return;
  const long v = px / hw, q = px % hw;
  if (mode == PW_DEPTH) {
    o0[px] = expf(acc[0]);
    o1[px] = 1.f + expf(acc[1]);
  } else if (mode == PW_RAY) {
    for (int o = 0; o < cout; ++o) o0[(v * cout + o) * hw + q] = acc[o];
  } else {
    if (o0)
      for (int o = 0; o < cout; ++o) o0[(v * cout + o) * hw + q] = acc[o];
    // mapanything-rs/src/model.rs:155-168
    const float nrm = fmaxf(sqrtf(acc[0] * acc[0] + acc[1] * acc[1] + acc[2] * acc[2]), 1e-8f);
    const float depth = expf(acc[3]) * (scale ? *scale : 1.f);
    if (o1) {
      o1[px * 3 + 0] = acc[0] / nrm * depth;
      o1[px * 3 + 1] = acc[1] / nrm * depth;
      o1[px * 3 + 2] = acc[2] / nrm * depth;
    }
    if (o2) o2[px] = 1.f + expf(acc[4]);
    if (o3) o3[px] = acc[5] > 0.f ? 1 : 0;
  }
}

// MapAnything head on 128-channel pixels: 8 lanes per pixel, each holding 16 channels and
// their 6x16 weights in registers (loaded once, then a grid-stride loop over pixels, two per
// lane group per trip so that two loads are in flight). The 6 dot products are summed across
// the 8 lanes with DPP (the two quad swaps, then the half-row mirror), which leaves all 6 sums
// in every lane, and the lanes share the pixel's stores.
template <typename T>
__global__ void __launch_bounds__(256) pw_ma128_kernel(const void* in, long pix, int hw, const float* w, const float* b,
                                                       float* o0, float* o1, float* o2, uint8_t* o3, const float* scale) {
  constexpr int UNROLL = 2;
  const int sub = threadIdx.x & 7, c0 = sub * 16;
  float wr[6][16];
#pragma unroll
  for (int o = 0; o < 6; ++o)
#pragma unroll
    for (int k = 0; k < 16; ++k) wr[o][k] = w[o * 128 + c0 + k];
  float bo[6];
#pragma unroll
  for (int o = 0; o < 6; ++o) bo[o] = b[o];
  const float sc = scale ? *scale : 1.f;
  const long groups = long(gridDim.x) * blockDim.x / 8;
  for (long base = (long(blockIdx.x) * blockDim.x + threadIdx.x) / 8; base < pix; base += groups * UNROLL) {
    float x[UNROLL][16];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const long px = base + u * groups;
#pragma unroll
      for (int k = 0; k < 16; k += 4) {
        const float4 f = px < pix ? ld4<T>(in, px * 128 + c0 + k) : make_float4(0.f, 0.f, 0.f, 0.f);
        x[u][k] = f.x; x[u][k + 1] = f.y; x[u][k + 2] = f.z; x[u][k + 3] = f.w;
      }
    }
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const long px = base + u * groups;
      float acc[6];
#pragma unroll
      for (int o = 0; o < 6; ++o) {
        float s = 0.f;
#pragma unroll
        for (int k = 0; k < 16; ++k) s += wr[o][k] * x[u][k];
        s = dpp_add<0xB1>(s);   // quad_perm [1,0,3,2]
        s = dpp_add<0x4E>(s);   // quad_perm [2,3,0,1]
        s = dpp_add<0x141>(s);  // row_half_mirror: the other quad of the 8
        acc[o] = s + bo[o];
      }
      if (px >= pix) continue;  // uniform across the pixel's 8 lanes
      const long v = px / hw, q = px - v * hw;
      float mine = acc[0];
#pragma unroll
      for (int o = 1; o < 6; ++o) mine = sub == o ? acc[o] : mine;
      if (o0 && sub < 6) o0[(v * 6 + sub) * hw + q] = mine;
      // mapanything-rs/src/model.rs:155-168
      const float nrm = fmaxf(sqrtf(acc[0] * acc[0] + acc[1] * acc[1] + acc[2] * acc[2]), 1e-8f);
      const float depth = expf(acc[3]) * sc;
      if (o1 && sub < 3) o1[px * 3 + sub] = mine / nrm * depth;
      if (o2 && sub == 6) o2[px] = 1.f + expf(acc[4]);
      if (o3 && sub == 7) o3[px] = acc[5] > 0.f ? 1 : 0;
    }
  }
}

void pointwise_head(const Exec& ex, int dt, int mode, const void* in, long pix, int hw, int cin, int cout,
                    const float* w, const float* b, float* o0, float* o1, float* o2, uint8_t* o3, const float* scale) {
  if (mode == PW_MA && cin == 128 && cout == 6 && !ex.dry && pix > 0 && (reinterpret_cast<uintptr_t>(in) & 15) == 0) {
    const double obytes = (o0 ? 24.0 : 0) + (o1 ? 12.0 : 0) + (o2 ? 4.0 : 0) + (o3 ? 1.0 : 0);
    ProfScope ps(ex, "pointwise_head", 2.0 * pix * cin * cout, double(pix) * (cin * dtype_size(dt) + obytes));
    // about three 256-thread blocks per CU, each lane group walking many pixels
    const long blocks = std::min<long>(cdiv(pix * 8, 256), 256L * 3);
    by_dt(dt, [&](auto t) {
      hipLaunchKernelGGL(pw_ma128_kernel<TY(t)>, dim3(blocks), dim3(256), 0, ex.stream, in, pix, hw, w, b, o0, o1, o2, o3, scale);
    });
    SPLAT_HIP(hipGetLastError());
    return;
  }
  if ((cin == 32 || cin == 64 || cin == 128) && !ex.dry && pix > 0 && cout <= 8 &&
      (reinterpret_cast<uintptr_t>(in) & 15) == 0) {
    SPLAT_CHECK(mode != PW_DEPTH || cout == 2, BAD_ARGUMENT, "depth head has 2 channels");
    SPLAT_CHECK(mode != PW_MA || cout == 6, BAD_ARGUMENT, "MapAnything head has 6 channels");
    const double obytes = mode == PW_MA ? (o0 ? 24.0 : 0) + (o1 ? 12.0 : 0) + (o2 ? 4.0 : 0) + (o3 ? 1.0 : 0) : 4.0 * cout;
    ProfScope ps(ex, "pointwise_head", 2.0 * pix * cin * cout, double(pix) * (cin * dtype_size(dt) + obytes));
    const int lpp = cin / 8;
    dim3 grid(cdiv(pix * lpp, 256));
#define PWC(T, L) hipLaunchKernelGGL((pw_coop_kernel<T, L>), grid, dim3(256), 0, ex.stream, mode, in, pix, hw, cin, cout, w, b, o0, o1, o2, o3, scale)
    by_dt(dt, [&](auto t) {
      if (lpp == 4) PWC(TY(t), 4); else if (lpp == 8) PWC(TY(t), 8); else PWC(TY(t), 16);
    });
#undef PWC
    SPLAT_HIP(hipGetLastError());
    return;
  }
  SPLAT_CHECK(cout <= 8 && cout * cin <= 8 * 256 && hw > 0, BAD_ARGUMENT, "pointwise_head sizes");
  SPLAT_CHECK(mode != PW_DEPTH || cout == 2, BAD_ARGUMENT, "depth head has 2 channels");
  SPLAT_CHECK(mode != PW_MA || cout == 6, BAD_ARGUMENT, "MapAnything head has 6 channels");
  if (ex.dry || pix == 0) return;
  const double obytes = mode == PW_MA ? (o0 ? 24.0 : 0) + (o1 ? 12.0 : 0) + (o2 ? 4.0 : 0) + (o3 ? 1.0 : 0) : 4.0 * cout;
  ProfScope ps(ex, "pointwise_head", 2.0 * pix * cin * cout, double(pix) * (cin * dtype_size(dt) + obytes));
  dim3 grid(cdiv(pix, 256));
  by_dt(dt, [&](auto t) {
    hipLaunchKernelGGL(pw_kernel<TY(t)>, grid, dim3(256), 0, ex.stream, mode, in, pix, hw, cin, cout, w, b, o0, o1, o2, o3, scale);
  });
  SPLAT_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------------------
// Small linears for the heads: one wave per output column n. Each lane takes 8 consecutive k
// at a time (one 16-byte weight load) and keeps the partial sums of up to 8 rows, so the weight
// row is read once for all rows.
template <typename TW> __device__ inline void load_w8(const void* W, long i, float* w) {  // the 16-bit types
  const uint4 u = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(W) + i);
  const uint32_t q[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    w[2 * k] = u16f<TW>(q[k]);
    w[2 * k + 1] = u16f<TW>(q[k] >> 16);
  }
}
template <> __device__ inline void load_w8<float>(const void* W, long i, float* w) {
  const float4 a = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(W) + i);
  const float4 b = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(W) + i + 4);
  w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w; w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
}

template <typename TW>
__global__ void small_linear8_kernel(const float* x, long ldx, int M, int K, const void* W, long ldw, const float* b,
                                     float* y, long ldy, int N, int act) {
  const int wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6, lane = threadIdx.x & 63;
  if (wave >= N) return;
  const long wb = (long)wave * ldw;
  for (int m0 = 0; m0 < M; m0 += 8) {
    float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int k = lane * 8; k < K; k += 512) {
      float w[8];
      load_w8<TW>(W, wb + k, w);
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        if (m0 + m < M) {
          const float4 a = *reinterpret_cast<const float4*>(x + long(m0 + m) * ldx + k);
          const float4 c = *reinterpret_cast<const float4*>(x + long(m0 + m) * ldx + k + 4);
          s[m] += w[0] * a.x + w[1] * a.y + w[2] * a.z + w[3] * a.w + w[4] * c.x + w[5] * c.y + w[6] * c.z + w[7] * c.w;
        }
      }
    }
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      if (m0 + m >= M) break;
      const float t = wave_sum(s[m]);
      if (lane == 0) {
        float v = t + (b ? b[wave] : 0.f);
        if (act == ACT_RELU) v = fmaxf(v, 0.f);
        y[long(m0 + m) * ldy + wave] = v;
      }
    }
  }
}

// Scalar form for strides or sizes the 8-wide form cannot take.
template <typename TW>
__global__ void small_linear_kernel(const float* x, long ldx, int M, int K, const void* W, long ldw, const float* b,
                                    float* y, long ldy, int N, int act) {
  const int wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6, lane = threadIdx.x & 63;
  if (wave >= N) return;
  const long wb = (long)wave * ldw;
  for (int m = 0; m < M; ++m) {
    float s = 0.f;
    for (int k = lane; k < K; k += 64) s += x[m * ldx + k] * ld<TW>(W, wb + k);
    s = wave_sum(s);
    if (lane == 0) {
      float v = s + (b ? b[wave] : 0.f);
      if (act == ACT_RELU) v = fmaxf(v, 0.f);
      y[m * ldy + wave] = v;
    }
  }
}

void small_linear(const Exec& ex, int wdt, const float* x, long ldx, int M, int K, const void* W, long ldw,
                  const float* b, float* y, long ldy, int N, int act) {
  SPLAT_CHECK(ldw >= K && ldx >= K && ldy >= N, BAD_ARGUMENT, "small_linear strides");
  if (ex.dry || M == 0) return;
  ProfScope ps(ex, "small_linear", 2.0 * M * N * K, double(N) * K * dtype_size(wdt) + 4.0 * M * (K + N));
  dim3 grid(cdiv(N, 4));
  const bool vec = K % 8 == 0 && ldx % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(W) & 15) == 0 && (ldw * dtype_size(wdt)) % 16 == 0;
  if (vec) {
    by_dt(wdt, [&](auto t) {
      hipLaunchKernelGGL(small_linear8_kernel<TY(t)>, grid, dim3(256), 0, ex.stream, x, ldx, M, K, W, ldw, b, y, ldy, N, act);
    });
  } else {
    by_dt(wdt, [&](auto t) {
      hipLaunchKernelGGL(small_linear_kernel<TY(t)>, grid, dim3(256), 0, ex.stream, x, ldx, M, K, W, ldw, b, y, ldy, N, act);
    });
  }
  SPLAT_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------------------
// depthanything3-rs/src/reference_view.rs:38-80 on the device, in f64: Gram matrix and row
// sums of the class tokens, then mean cosine similarity, norm and unbiased variance of the
// unit token, each min-max scaled, balance = sum |x - 0.5|, first argmin. Up to REF_MAX_VIEWS
// views one block holds the Gram matrix in shared memory; beyond that one block per view
// computes its metrics (the same dot products, sums and order, so the same bits) into the
// workspace and one more block scales them and takes the argmin.
constexpr int REF_MAX_VIEWS = 64;

// Sum over the lanes of a dot product of two dim-long rows (lane-strided, then the wave sum).
__device__ inline double row_dot_d(const float* a, const float* b, int dim, int lane) {
  double s = 0.0;
  for (int c = lane; c < dim; c += 64) s += double(a[c]) * double(b[c]);
  return wave_sum_d(s);
}

__global__ void __launch_bounds__(1024) ref_view_kernel(const float* xs, int V, int n, int dim, int strategy, int* ref) {
  __shared__ double gram[REF_MAX_VIEWS * REF_MAX_VIEWS];
  __shared__ double rsum[REF_MAX_VIEWS];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  if (V < 3 || strategy == 0) {
    if (threadIdx.x == 0) *ref = 0;
    return;
  }
  if (strategy == 1) {
    if (threadIdx.x == 0) *ref = V / 2;
    return;
  }
  // the V(V+1)/2 pairs j >= i of the Gram matrix, then the V row sums, one wave each
  const int npair = V * (V + 1) / 2;
  for (int pq = wave; pq < npair + V; pq += nw) {
    double s = 0.0;
    if (pq < npair) {
      int i = 0, r = pq;
      while (r >= V - i) { r -= V - i; ++i; }
      const int j = i + r;
      const float* a = xs + (long)i * n * dim;
      const float* b = xs + (long)j * n * dim;
      for (int c = lane; c < dim; c += 64) s += double(a[c]) * double(b[c]);
      s = wave_sum_d(s);
      if (lane == 0) { gram[i * V + j] = s; gram[j * V + i] = s; }
    } else {
      const int i = pq - npair;
      const float* a = xs + (long)i * n * dim;
      for (int c = lane; c < dim; c += 64) s += double(a[c]);
      s = wave_sum_d(s);
      if (lane == 0) rsum[i] = s;
    }
  }
  __syncthreads();
  // Per-view metrics, one thread per view (the reference's loops over j in the same order)
  __shared__ double met[3][REF_MAX_VIEWS];
  __shared__ double lohi[3][2];
  __shared__ double bal[REF_MAX_VIEWS];
  const int i = threadIdx.x;
  if (i < V) {
    const double nrm = sqrt(gram[i * V + i]);
    double s = 0.0;
    for (int j = 0; j < V; ++j)
      if (j != i) s += gram[i * V + j] / (nrm * sqrt(gram[j * V + j]));
    const double mean = rsum[i] / nrm / dim;
    const double sq = gram[i * V + i] / (nrm * nrm);
    met[0][i] = s / (V - 1);
    met[1][i] = nrm;
    met[2][i] = (sq - dim * mean * mean) / (dim - 1);
  }
  __syncthreads();
  if (i < 3) {  // min-max range of metric i over the views
    double lo = INFINITY, hi = -INFINITY;
    for (int v = 0; v < V; ++v) { lo = fmin(lo, met[i][v]); hi = fmax(hi, met[i][v]); }
    lohi[i][0] = lo;
    lohi[i][1] = hi;
  }
  __syncthreads();
  if (i < V) {
    double b = 0.0;
    for (int k = 0; k < 3; ++k) b += fabs((met[k][i] - lohi[k][0]) / (lohi[k][1] - lohi[k][0] + 1e-8) - 0.5);
    bal[i] = b;
  }
  __syncthreads();
  if (i == 0) {  // the first argmin
    int best = 0;
    for (int v = 1; v < V; ++v)
      if (bal[v] < bal[best]) best = v;
    *ref = best;
  }
}

// Block i: view i's mean cosine similarity, norm and variance into met[0 / V / 2V + i]. The
// similarity terms of REF_CHUNK views at a time go through shared memory and thread 0 adds
// them in view order, skipping i.
constexpr int REF_CHUNK = 256;

__global__ void __launch_bounds__(256) ref_view_metrics_kernel(const float* xs, int V, int n, int dim, double* met) {
  __shared__ double term[REF_CHUNK];
  __shared__ double own[2];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const int i = blockIdx.x;
  const float* a = xs + (long)i * n * dim;
  if (wave == 0) {
    const double g = row_dot_d(a, a, dim, lane);
    if (lane == 0) own[0] = g;
  } else if (wave == 1) {
    double r = 0.0;
    for (int c = lane; c < dim; c += 64) r += double(a[c]);
    r = wave_sum_d(r);
    if (lane == 0) own[1] = r;
  }
  __syncthreads();
  const double nrm = sqrt(own[0]);
  double s = 0.0;
  for (int j0 = 0; j0 < V; j0 += REF_CHUNK) {
    const int cnt = min(REF_CHUNK, V - j0);
    for (int t = wave; t < cnt; t += nw) {
      const int j = j0 + t;
      const float* b = xs + (long)j * n * dim;
      const double gij = row_dot_d(a, b, dim, lane);
      const double gjj = row_dot_d(b, b, dim, lane);
      if (lane == 0) term[t] = gij / (nrm * sqrt(gjj));
    }
    __syncthreads();
    if (threadIdx.x == 0)
      for (int t = 0; t < cnt; ++t)
        if (j0 + t != i) s += term[t];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const double mean = own[1] / nrm / dim;
    const double sq = own[0] / (nrm * nrm);
    met[i] = s / (V - 1);
    met[V + i] = nrm;
    met[2 * V + i] = (sq - dim * mean * mean) / (dim - 1);
  }
}

// Min-max range of each metric (three threads), then the balance and its first argmin in
// view order (thread 0).
__global__ void __launch_bounds__(64) ref_view_pick_kernel(const double* met, int V, int* ref) {
  __shared__ double lohi[3][2];
  const int k = threadIdx.x;
  if (k < 3) {
    double lo = INFINITY, hi = -INFINITY;
    for (int v = 0; v < V; ++v) { lo = fmin(lo, met[k * V + v]); hi = fmax(hi, met[k * V + v]); }
    lohi[k][0] = lo;
    lohi[k][1] = hi;
  }
  __syncthreads();
  if (k == 0) {
    int best = 0;
    double best_b = 0.0;
    for (int v = 0; v < V; ++v) {
      double b = 0.0;
      for (int m = 0; m < 3; ++m) b += fabs((met[m * V + v] - lohi[m][0]) / (lohi[m][1] - lohi[m][0] + 1e-8) - 0.5);
      if (v == 0 || b < best_b) {
        best = v;
        best_b = b;
      }
    }
    *ref = best;
  }
}

void select_reference_view(const Exec& ex, const float* xs, int V, int n, int dim, int strategy, int* ref) {
  SPLAT_CHECK(V >= 1 && n >= 1 && dim >= 2, BAD_SHAPE, "reference-view selection: bad token shape");
  const bool grid = V > REF_MAX_VIEWS && V >= 3 && strategy == 2;
  const size_t bytes = size_t(3) * V * sizeof(double);
  if (ex.dry) {
    if (grid && ex.ws) ex.ws->need = std::max(ex.ws->need, bytes);
    return;
  }
  if (!grid) {  // beyond REF_MAX_VIEWS only the fixed choices (first, middle) reach this kernel
    hipLaunchKernelGGL(ref_view_kernel, dim3(1), dim3(1024), 0, ex.stream, xs, V, n, dim, strategy, ref);
    SPLAT_HIP(hipGetLastError());
    return;
  }
  SPLAT_CHECK(ex.ws && ex.ws->ptr && ex.ws->cap >= bytes, BAD_ARGUMENT,
              "reference-view selection over more than 64 views needs the sized workspace");
  double* met = static_cast<double*>(ex.ws->ptr);
  hipLaunchKernelGGL(ref_view_metrics_kernel, dim3(V), dim3(256), 0, ex.stream, xs, V, n, dim, met);
  hipLaunchKernelGGL(ref_view_pick_kernel, dim3(1), dim3(64), 0, ex.stream, met, V, ref);
  SPLAT_HIP(hipGetLastError());
}

__global__ void camera_tokens_kernel(float* xs, int V, int n, int dim, const float* cam, const int* ref) {
  const long id = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= (long)V * dim) return;
  const int v = int(id / dim), c = int(id % dim);
  xs[(long)v * n * dim + c] = cam[(v == *ref ? 0 : dim) + c];
}

void set_camera_tokens(const Exec& ex, float* xs, int V, int n, int dim, const float* cam, const int* ref) {
  if (ex.dry) return;
  hipLaunchKernelGGL(camera_tokens_kernel, dim3(cdiv((long)V * dim, 256)), dim3(256), 0, ex.stream, xs, V, n, dim, cam, ref);
  SPLAT_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------------------
// depthanything3-rs/src/backbone.rs:177-189 + the dense head's input norm (dpt.rs:277).
// One wave per token: the row of the current output (xs) and of the layer output kept
// (within) are read once, as float2 runs of 128 channels per wave (dim is a multiple of 128 in
// every DA3 variant, at most HOOK_RUNS * 128), and both norms are taken from registers.
constexpr int HOOK_RUNS = 12;
template <typename T>
__global__ void __launch_bounds__(256) da3_hook_kernel(const float* within, const float* xs, int V, int n, int dim,
                                                       const float* bnw, const float* bnb, const float* hnw,
                                                       const float* hnb, void* out, float* cam_out) {
  const long wave = ((long)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (wave >= (long)V * n) return;
  const int v = int(wave / n), t = int(wave % n);
  const float* a = xs + wave * dim;
  const float* w = within + wave * dim;
  if (t == 0) {
    if (cam_out)
      for (int c = lane; c < dim; c += 64) {
        cam_out[(long)v * 2 * dim + c] = w[c];
        cam_out[(long)v * 2 * dim + dim + c] = a[c];
      }
    return;
  }
  const int runs = dim >> 7;
  float2 av[HOOK_RUNS], wv[HOOK_RUNS];
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < HOOK_RUNS; ++k)
    if (k < runs) {
      av[k] = *reinterpret_cast<const float2*>(a + k * 128 + 2 * lane);
      wv[k] = *reinterpret_cast<const float2*>(w + k * 128 + 2 * lane);
      s += av[k].x + av[k].y;
    }
  // backbone norm of the current output (eps 1e-5)
  const float am = wave_sum(s) / dim;
  float q = 0.f;
#pragma unroll
  for (int k = 0; k < HOOK_RUNS; ++k)
    if (k < runs) {
      const float d0 = av[k].x - am, d1 = av[k].y - am;
      q += d0 * d0 + d1 * d1;
    }
  const float ar = rsqrtf(wave_sum(q) / dim + 1e-5f);
  // head norm over cat(within, normed) (eps 1e-5); av becomes the normed output
  s = 0.f;
#pragma unroll
  for (int k = 0; k < HOOK_RUNS; ++k)
    if (k < runs) {
      const int c = k * 128 + 2 * lane;
      av[k].x = (av[k].x - am) * ar * bnw[c] + bnb[c];
      av[k].y = (av[k].y - am) * ar * bnw[c + 1] + bnb[c + 1];
      s += wv[k].x + wv[k].y + av[k].x + av[k].y;
    }
  const float hm = wave_sum(s) / (2 * dim);
  q = 0.f;
#pragma unroll
  for (int k = 0; k < HOOK_RUNS; ++k)
    if (k < runs) {
      const float d0 = wv[k].x - hm, d1 = wv[k].y - hm, d2 = av[k].x - hm, d3 = av[k].y - hm;
      q += d0 * d0 + d1 * d1 + d2 * d2 + d3 * d3;
    }
  const float hr = rsqrtf(wave_sum(q) / (2 * dim) + 1e-5f);
  const long ob = ((long)v * (n - 1) + t - 1) * 2 * dim;
#pragma unroll
  for (int k = 0; k < HOOK_RUNS; ++k)
    if (k < runs) {
      const int c = k * 128 + 2 * lane;
      st<T>(out, ob + c, (wv[k].x - hm) * hr * hnw[c] + hnb[c]);
      st<T>(out, ob + c + 1, (wv[k].y - hm) * hr * hnw[c + 1] + hnb[c + 1]);
      st<T>(out, ob + dim + c, (av[k].x - hm) * hr * hnw[dim + c] + hnb[dim + c]);
      st<T>(out, ob + dim + c + 1, (av[k].y - hm) * hr * hnw[dim + c + 1] + hnb[dim + c + 1]);
    }
}

void da3_hook(const Exec& ex, int dt, const float* within, const float* xs, int V, int n, int dim, const float* bnw,
              const float* bnb, const float* hnw, const float* hnb, void* out, float* cam_out) {
  SPLAT_CHECK(dim % 128 == 0 && dim <= HOOK_RUNS * 128, BAD_SHAPE, "da3_hook: dim must be a multiple of 128, at most 1536");
  if (ex.dry) return;
  ProfScope ps(ex, "da3_hook", 0, double(V) * n * dim * 8 + double(V) * (n - 1) * 2 * dim * dtype_size(dt));
  dim3 grid(cdiv((long)V * n, 4));
  by_dt(dt, [&](auto t) {
    hipLaunchKernelGGL(da3_hook_kernel<TY(t)>, grid, dim3(256), 0, ex.stream, within, xs, V, n, dim, bnw, bnb, hnw, hnb, out, cam_out);
  });
  SPLAT_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------------------
template <typename TI, typename TO>
__global__ void convert_kernel(const void* in, void* out, long count) {
  const long id = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (id < count) st<TO>(out, id, ld<TI>(in, id));
}

void convert(const Exec& ex, int in_dt, const void* in, int out_dt, void* out, long count) {
  if (ex.dry || count == 0) return;
  dim3 grid(cdiv(count, 256));
  SPLAT_CHECK(in_dt_ok(in_dt) && in_dt_ok(out_dt), BAD_ARGUMENT, "convert: dtype");
  by_dt(in_dt, [&](auto ti) {
    by_dt(out_dt, [&](auto to) {
      hipLaunchKernelGGL((convert_kernel<TY(ti), TY(to)>), grid, dim3(256), 0, ex.stream, in, out, count);
    });
  });
  SPLAT_HIP(hipGetLastError());
}

template <typename TI, typename TO>
__global__ void convert_rows_kernel(const void* in, long ldi, void* out, long ldo, int rows, int cols) {
  const long id = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= (long)rows * cols) return;
  const long r = id / cols, c = id - r * cols;
  st<TO>(out, r * ldo + c, ld<TI>(in, r * ldi + c));
}

void convert_rows(const Exec& ex, int in_dt, const void* in, long ldi, int out_dt, void* out, long ldo, int rows,
                  int cols) {
  if (ex.dry || rows == 0 || cols == 0) return;
  SPLAT_CHECK(in_dt_ok(in_dt) && in_dt_ok(out_dt), BAD_ARGUMENT, "convert_rows: dtype");
  dim3 grid(cdiv((long)rows * cols, 256));
  by_dt(in_dt, [&](auto ti) {
    by_dt(out_dt, [&](auto to) {
      hipLaunchKernelGGL((convert_rows_kernel<TY(ti), TY(to)>), grid, dim3(256), 0, ex.stream, in, ldi, out, ldo, rows,
                         cols);
    });
  });
  SPLAT_HIP(hipGetLastError());
}

__global__ void add_rows_kernel(float* xs, int rows, int dim, const float* vec) {
  const long id = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (id < (long)rows * dim) xs[id] += vec[id % dim];
}

void add_rows(const Exec& ex, float* xs, int rows, int dim, const float* vec) {
  if (ex.dry || rows == 0) return;
  hipLaunchKernelGGL(add_rows_kernel, dim3(cdiv((long)rows * dim, 256)), dim3(256), 0, ex.stream, xs, rows, dim, vec);
  SPLAT_HIP(hipGetLastError());
}

// One thread per pixel: the unit direction ((x - cx)/fx, (y - cy)/fy, 1)/norm in f64
// (mapanything-rs/src/model.rs:42-50), stored as f32 at its pixel-unshuffled position.
__global__ void ray_unshuffled_kernel(const double* cam, int V, int H, int W, float* out) {
  const long id = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long hw = (long)H * W;
  if (id >= (long)V * hw) return;
  const int v = int(id / hw), pix = int(id - v * hw), y = pix / W, x = pix - y * W;
  const double* c = cam + v * 5;
  const double dx = (double(x) - c[2]) / c[0], dy = (double(y) - c[3]) / c[1];
  const double inv = 1.0 / sqrt(dx * dx + dy * dy + 1.0);
  const int R = H / 14, C = W / 14, r = y / 14, i = y - r * 14, col = x / 14, j = x - col * 14;
  float* o = out + ((long(v) * R + r) * C + col) * 588 + i * 14 + j;
  o[0] = float(dx * inv);
  o[196] = float(dy * inv);
  o[392] = float(inv);
}

void ray_unshuffled(const Exec& ex, const double* cam, int V, int H, int W, float* out) {
  if (ex.dry || V == 0) return;
  SPLAT_CHECK(H % 14 == 0 && W % 14 == 0, BAD_SHAPE, "ray map: H and W must be multiples of 14");
  ProfScope ps(ex, "ray_map", 0.0, double(V) * H * W * 12);
  hipLaunchKernelGGL(ray_unshuffled_kernel, dim3(cdiv((long)V * H * W, 256)), dim3(256), 0, ex.stream, cam, V, H, W,
                     out);
  SPLAT_HIP(hipGetLastError());
}

__global__ void add_view_features_kernel(float* xs, int V, int n, int P, int dim, const float* feat,
                                         const double* cam) {
  const long id = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= (long)V * P * dim) return;
  const long row = id / dim;
  const int v = int(row / P), p = int(row - long(v) * P), c = int(id - row * dim);
  if (cam[v * 5 + 4] != 0.0) xs[(long(v) * n + 1 + p) * dim + c] += feat[id];
}

void add_view_features(const Exec& ex, float* xs, int V, int n, int P, int dim, const float* feat, const double* cam) {
  if (ex.dry || V == 0) return;
  hipLaunchKernelGGL(add_view_features_kernel, dim3(cdiv((long)V * P * dim, 256)), dim3(256), 0, ex.stream, xs, V, n,
                     P, dim, feat, cam);
  SPLAT_HIP(hipGetLastError());
}

__global__ void copy_rows_kernel(float* dst, long lddst, const float* src, long ldsrc, int rows, int dim) {
  const long id = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= (long)rows * dim) return;
  const long r = id / dim, c = id % dim;
  dst[r * lddst + c] = src[r * ldsrc + c];
}

void copy_rows_f32(const Exec& ex, float* dst, long lddst, const float* src, long ldsrc, int rows, int dim) {
  if (ex.dry || rows == 0) return;
  hipLaunchKernelGGL(copy_rows_kernel, dim3(cdiv((long)rows * dim, 256)), dim3(256), 0, ex.stream, dst, lddst, src, ldsrc, rows, dim);
  SPLAT_HIP(hipGetLastError());
}

// Block (group, 64-column chunk): the 4 waves stride over the P rows, lanes over columns,
// then the 4 partial sums meet in LDS.
// Mean over the P rows of each group, in two passes: blocks of (group, 512 channels, slice of
// P/8 rows) sum 8-channel vectors into per-slice partials (4 row lanes per block, reduced in
// LDS), then one thread per (group, channel) adds the 8 partials in order. The partials live in
// the context workspace. A single pass (one block per 64 channels walking all P rows) took
// 68 us at C4 for 12.7 MB.
constexpr int MEAN_SLICES = 8;
template <typename T>
__global__ void __launch_bounds__(256) mean_rows_part_kernel(const void* in, int P, int C, float* part) {
  __shared__ float red[4][64 * 8];
  const int g = blockIdx.x, lane = threadIdx.x & 63, rl = threadIdx.x >> 6;
  const int c = (blockIdx.y * 64 + lane) * 8;
  const int chunk = (P + MEAN_SLICES - 1) / MEAN_SLICES, p0 = blockIdx.z * chunk, p1 = min(P, p0 + chunk);
  float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (c < C)
    for (int p = p0 + rl; p < p1; p += 4) {
      float v[8];
      Vec8<T>::load(in, (long(g) * P + p) * C + c, v);
#pragma unroll
      for (int k = 0; k < 8; ++k) s[k] += v[k];
    }
#pragma unroll
  for (int k = 0; k < 8; ++k) red[rl][lane * 8 + k] = s[k];
  __syncthreads();
  if (rl == 0 && c < C) {
    float* dst = part + (long(blockIdx.z) * gridDim.x + g) * C + c;
#pragma unroll
    for (int k = 0; k < 8; ++k) dst[k] = (red[0][lane * 8 + k] + red[1][lane * 8 + k]) + (red[2][lane * 8 + k] + red[3][lane * 8 + k]);
  }
}
__global__ void mean_rows_final_kernel(const float* part, int groups, int P, int C, float* out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= groups * C) return;
  float s = 0.f;
  for (int r = 0; r < MEAN_SLICES; ++r) s += part[long(r) * groups * C + i];
  out[i] = s / P;
}

template <typename T>
__global__ void mean_rows_kernel(const void* in, int groups, int P, int C, float* out) {
  __shared__ float part[4][64];
  const int gi = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = blockIdx.y * 64 + lane;
  float s = 0.f;
  if (c < C)
    for (int p = wave; p < P; p += 4) s += ld<T>(in, ((long)gi * P + p) * C + c);
  part[wave][lane] = s;
  __syncthreads();
  if (wave == 0 && c < C) out[(long)gi * C + c] = (part[0][lane] + part[1][lane] + part[2][lane] + part[3][lane]) / P;
}

void mean_rows(const Exec& ex, int dt, const void* in, int groups, int P, int C, float* out) {
  const size_t pbytes = size_t(MEAN_SLICES) * groups * C * sizeof(float);
  const bool two_pass = C % 8 == 0 && (reinterpret_cast<uintptr_t>(in) & 15) == 0 && ex.ws;
  if (ex.dry) {
    if (two_pass) ex.ws->need = std::max(ex.ws->need, pbytes);
    return;
  }
  ProfScope ps(ex, "mean_rows", 0, double(groups) * P * C * dtype_size(dt) + 4.0 * groups * C);
  if (two_pass && ex.ws->ptr && ex.ws->cap >= pbytes) {
    float* part = static_cast<float*>(ex.ws->ptr);
    dim3 grid(groups, cdiv(C / 8, 64), MEAN_SLICES);
    by_dt(dt, [&](auto t) { hipLaunchKernelGGL(mean_rows_part_kernel<TY(t)>, grid, dim3(256), 0, ex.stream, in, P, C, part); });
    SPLAT_HIP(hipGetLastError());
    hipLaunchKernelGGL(mean_rows_final_kernel, dim3(cdiv(groups * C, 256)), dim3(256), 0, ex.stream, part, groups, P, C, out);
    SPLAT_HIP(hipGetLastError());
    return;
  }
  dim3 grid(groups, cdiv(C, 64));
  by_dt(dt, [&](auto t) { hipLaunchKernelGGL(mean_rows_kernel<TY(t)>, grid, dim3(256), 0, ex.stream, in, groups, P, C, out); });
  SPLAT_HIP(hipGetLastError());
}

__global__ void exp_clamp_kernel(float* x, int count, float lo) {
  const int id = blockIdx.x * blockDim.x + threadIdx.x;
  if (id < count) x[id] = fmaxf(expf(x[id]), lo);
}
void exp_clamp(const Exec& ex, float* x, int count, float lo) {
  if (ex.dry) return;
  hipLaunchKernelGGL(exp_clamp_kernel, dim3(cdiv(count, 256)), dim3(256), 0, ex.stream, x, count, lo);
  SPLAT_HIP(hipGetLastError());
}

__global__ void normalize_rows_kernel(float* x, int rows, int dim, float min_norm) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  float s = 0.f;
  for (int c = 0; c < dim; ++c) s += x[r * dim + c] * x[r * dim + c];
  const float nrm = fmaxf(sqrtf(s), min_norm);
  for (int c = 0; c < dim; ++c) x[r * dim + c] /= nrm;
}
void normalize_rows(const Exec& ex, float* x, int rows, int dim, float min_norm) {
  if (ex.dry) return;
  hipLaunchKernelGGL(normalize_rows_kernel, dim3(cdiv(rows, 64)), dim3(64), 0, ex.stream, x, rows, dim, min_norm);
  SPLAT_HIP(hipGetLastError());
}

__global__ void scale_rows_kernel(const float* x, int count, const float* scale, float* out) {
  const int id = blockIdx.x * blockDim.x + threadIdx.x;
  if (id < count) out[id] = x[id] * *scale;
}
void scale_rows(const Exec& ex, const float* x, int rows, int dim, const float* scale, float* out) {
  if (ex.dry) return;
  hipLaunchKernelGGL(scale_rows_kernel, dim3(cdiv(rows * dim, 256)), dim3(256), 0, ex.stream, x, rows * dim, scale, out);
  SPLAT_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------------------
// Post-forward geometry (depthanything3-rs/src/pipeline.rs:44-133, mapanything-rs/src/
// {pipeline.rs:18-104, reconstruction.rs:22-33, cleaning.rs:28-64}), in f64 like the
// reference's nalgebra code. cam [V, 16] f64 per view: camera -> view-0 frame rotation R
// (row-major), translation t, focal (fx, fy), principal point (cx, cy).

__device__ inline void quat_rotation(double x, double y, double z, double w, double* R) {
  const double n = sqrt(x * x + y * y + z * z + w * w);  // UnitQuaternion::from_quaternion normalises
  x /= n; y /= n; z /= n; w /= n;
  R[0] = 1 - 2 * (y * y + z * z); R[1] = 2 * (x * y - z * w);     R[2] = 2 * (x * z + y * w);
  R[3] = 2 * (x * y + z * w);     R[4] = 1 - 2 * (x * x + z * z); R[5] = 2 * (y * z - x * w);
  R[6] = 2 * (x * z - y * w);     R[7] = 2 * (y * z + x * w);     R[8] = 1 - 2 * (x * x + y * y);
}

// One thread per view. DA3 (pose_enc != NULL): t, xyzw quaternion, fov_h, fov_w
// (camera_head.rs:28-53); MapAnything: quaternion, metric translation and the fitted
// intrinsics (fitted [V, 4] = cx, cy, fx, fy). Poses are re-expressed relative to view 0
// (reconstruction.rs:22-33): R0^T R, R0^T (t - t0).
__global__ void recon_cameras_kernel(int V, int H, int W, const float* pose_enc, const float* quat, const float* trans,
                                     const double* fitted, double* cam) {
  const int v = blockIdx.x * blockDim.x + threadIdx.x;
  if (v >= V) return;
  double R[9], R0[9], t[3], t0[3];
  auto pose = [&](int u, double* Ru, double* tu) {
    if (pose_enc) {
      const float* e = pose_enc + u * 9;
      quat_rotation(e[3], e[4], e[5], e[6], Ru);
      for (int k = 0; k < 3; ++k) tu[k] = e[k];
    } else {
      const float* q = quat + u * 4;
      quat_rotation(q[0], q[1], q[2], q[3], Ru);
      for (int k = 0; k < 3; ++k) tu[k] = trans[u * 3 + k];
    }
  };
  pose(v, R, t);
  pose(0, R0, t0);
  double* c = cam + v * 16;
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 3; ++j) c[i * 3 + j] = R0[0 * 3 + i] * R[0 * 3 + j] + R0[1 * 3 + i] * R[1 * 3 + j] + R0[2 * 3 + i] * R[2 * 3 + j];
  for (int i = 0; i < 3; ++i)
    c[9 + i] = R0[0 * 3 + i] * (t[0] - t0[0]) + R0[1 * 3 + i] * (t[1] - t0[1]) + R0[2 * 3 + i] * (t[2] - t0[2]);
  if (pose_enc) {
    const double fov_h = pose_enc[v * 9 + 7], fov_w = pose_enc[v * 9 + 8];
    c[12] = W / 2.0 / fmax(tan(fov_w / 2.0), 1e-6);
    c[13] = H / 2.0 / fmax(tan(fov_h / 2.0), 1e-6);
    c[14] = W / 2.0;
    c[15] = H / 2.0;
  } else {
    c[12] = fitted[v * 4 + 2];
    c[13] = fitted[v * 4 + 3];
    c[14] = fitted[v * 4 + 0];
    c[15] = fitted[v * 4 + 1];
  }
}

// One block per view: least squares pixel = centre + focal * coordinate / z per axis over
// every (side/50)-th pixel (mapanything-rs/src/pipeline.rs:18-39); out [V, 4] = cx, cy, fx, fy.
__global__ void __launch_bounds__(256) fit_intrinsics_kernel(const float* pts, int H, int W, double* out) {
  const int v = blockIdx.x;
  const int sy = max(H / 50, 1), sx = max(W / 50, 1);
  const int ny = (H + sy - 1) / sy, nx = (W + sx - 1) / sx;
  double acc[10] = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0};  // per axis: n, sum r, sum r^2, sum pix, sum r*pix
  for (int s = threadIdx.x; s < ny * nx; s += 256) {
    const int y = (s / nx) * sy, x = (s % nx) * sx;
    const float* p = pts + ((long(v) * H + y) * W + x) * 3;
    const double z = p[2];
    const double rx = double(p[0]) / z, ry = double(p[1]) / z;
    acc[0] += 1; acc[1] += rx; acc[2] += rx * rx; acc[3] += x; acc[4] += rx * x;
    acc[5] += 1; acc[6] += ry; acc[7] += ry * ry; acc[8] += y; acc[9] += ry * y;
  }
  __shared__ double red[10][256];
  for (int k = 0; k < 10; ++k) red[k][threadIdx.x] = acc[k];
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (threadIdx.x < w)
      for (int k = 0; k < 10; ++k) red[k][threadIdx.x] += red[k][threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x < 2) {
    const int a = threadIdx.x * 5;
    const double n = red[a][0], sr = red[a + 1][0], srr = red[a + 2][0], sp = red[a + 3][0], srp = red[a + 4][0];
    const double det = n * srr - sr * sr;
    out[v * 4 + threadIdx.x] = (sp * srr - sr * srp) / det;      // centre
    out[v * 4 + 2 + threadIdx.x] = (n * srp - sr * sp) / det;    // focal
  }
}

// One thread per pixel: camera-frame point (DA3: unprojected depth, pipeline.rs:44-51;
// MapAnything: the network's point) -> view-0 frame, R p + t, stored f32. conf0 = the
// confidence before cleaning (MapAnything: 0 where the mask calls the pixel ambiguous).
__global__ void unproject_kernel(int V, int H, int W, const float* depth, const float* pts_cam, const float* conf,
                                 const uint8_t* mask, const double* cam, float* points, float* conf0) {
  const long id = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long hw = (long)H * W;
  if (id >= V * hw) return;
  const int v = int(id / hw), pix = int(id - v * hw), y = pix / W, x = pix - y * W;
  const double* c = cam + v * 16;
  double p[3];
  if (depth) {
    const double d = depth[id];
    p[0] = (x - c[14]) / c[12] * d;
    p[1] = (y - c[15]) / c[13] * d;
    p[2] = d;
  } else {
    for (int k = 0; k < 3; ++k) p[k] = pts_cam[id * 3 + k];
  }
  for (int i = 0; i < 3; ++i) points[id * 3 + i] = float(c[i * 3] * p[0] + c[i * 3 + 1] * p[1] + c[i * 3 + 2] * p[2] + c[9 + i]);
  conf0[id] = mask && !mask[id] ? 0.f : conf[id];
}

// One thread per pixel of image i: zero its confidence if, seen from another view j, it lies
// in front (by more than 2%) of j's foreground depth at the pixel it projects to and is less
// confident (cleaning.rs:28-64). Projections use the view's mean focal; pixels round half
// away from zero (f64::round). Reads conf0 only, so every comparison sees the originals.
__global__ void clean_kernel(int V, int H, int W, const float* points, const float* conf0, const float* depth,
                             int dstride, const uint8_t* fg, const double* cam, float* conf) {
  const long id = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long hw = (long)H * W;
  if (id >= V * hw) return;
  const int i = int(id / hw);
  const float ci = conf0[id];
  bool zero = false;
  if (!fg || fg[id]) {
    const double px = points[id * 3], py = points[id * 3 + 1], pz = points[id * 3 + 2];
    for (int j = 0; j < V && !zero; ++j) {
      if (j == i) continue;
      const double* c = cam + j * 16;
      const double dx = px - c[9], dy = py - c[10], dz = pz - c[11];
      const double qx = c[0] * dx + c[3] * dy + c[6] * dz;   // R^T (p - t)
      const double qy = c[1] * dx + c[4] * dy + c[7] * dz;
      const double qz = c[2] * dx + c[5] * dy + c[8] * dz;
      if (!(qz > 0.0)) continue;
      const double f = (c[12] + c[13]) / 2.0;
      const double u = round(f * qx / qz + c[14]), vv = round(f * qy / qz + c[15]);
      if (!(u >= 0.0 && vv >= 0.0 && u < double(W) && vv < double(H))) continue;
      const long op = long(j) * hw + long(vv) * W + long(u);
      if ((!fg || fg[op]) && qz < (1.0 - 0.02) * double(depth[op * dstride]) && ci < conf0[op]) zero = true;
    }
  }
  conf[id] = zero ? 0.f : ci;
}

void reconstruct_geometry(const Exec& ex, int V, int H, int W, const float* depth, const float* pose_enc,
                          const float* pts_cam, const float* quat, const float* trans, const float* conf,
                          const uint8_t* mask, const uint8_t* fg, double* cam, double* fitted, float* conf0,
                          float* points, float* conf_out) {
  if (ex.dry || V == 0) return;
  const bool da3 = depth != nullptr;
  SPLAT_CHECK(da3 ? pose_enc != nullptr : (pts_cam && quat && trans && fitted), BAD_ARGUMENT, "geometry inputs");
  const long px = long(V) * H * W;
  ProfScope ps(ex, "geometry", 0.0, double(px) * (da3 ? 4 : 12) * 2 + double(px) * 4 * (V + 2) + double(px) * 12);
  if (!da3) hipLaunchKernelGGL(fit_intrinsics_kernel, dim3(V), dim3(256), 0, ex.stream, pts_cam, H, W, fitted);
  hipLaunchKernelGGL(recon_cameras_kernel, dim3(cdiv(V, 64)), dim3(64), 0, ex.stream, V, H, W, pose_enc, quat, trans,
                     fitted, cam);
  hipLaunchKernelGGL(unproject_kernel, dim3(cdiv(px, 256)), dim3(256), 0, ex.stream, V, H, W, depth, pts_cam, conf,
                     mask, cam, points, conf0);
  hipLaunchKernelGGL(clean_kernel, dim3(cdiv(px, 256)), dim3(256), 0, ex.stream, V, H, W, points, conf0,
                     da3 ? depth : pts_cam + 2, da3 ? 1 : 3, fg, cam, conf_out);
  SPLAT_HIP(hipGetLastError());
}

// mapanything-rs/src/image_input.rs:195-216 (to_model_input) for V images of one size:
// RGBA u8 [V, H, W, 4] -> ImageNet-normalised [V, 3, H, W] f32 ((x * (1/255) - mean) / std,
// candle's affine then broadcast ops, in that order) and foreground = alpha >= 128
// (FOREGROUND_MIN_ALPHA, image_input.rs:22).
__global__ void to_model_input_kernel(const uint8_t* rgba, int V, long hw, float* img, uint8_t* fg) {
  const long id = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= V * hw) return;
  const long v = id / hw, p = id - v * hw;
  const uchar4 px = reinterpret_cast<const uchar4*>(rgba)[id];
  const float mean[3] = {0.485f, 0.456f, 0.406f}, stdv[3] = {0.229f, 0.224f, 0.225f};
  const float scale = float(1.0 / 255.0);
  const float c[3] = {float(px.x), float(px.y), float(px.z)};
  for (int k = 0; k < 3; ++k) img[(v * 3 + k) * hw + p] = (c[k] * scale + 0.0f - mean[k]) / stdv[k];
  if (fg) fg[id] = px.w >= 128 ? 1 : 0;
}

void to_model_input(const Exec& ex, const uint8_t* rgba, int V, int H, int W, float* img, uint8_t* fg) {
  if (ex.dry || V == 0) return;
  const long hw = long(H) * W;
  hipLaunchKernelGGL(to_model_input_kernel, dim3(cdiv(V * hw, 256)), dim3(256), 0, ex.stream, rgba, V, hw, img, fg);
  SPLAT_HIP(hipGetLastError());
}

// image_input.rs:196-197: whether view v keeps a foreground pixel (alpha >= 128) after cropping.
// One block per view; every thread stops at its first foreground pixel, the block ORs them and
// thread 0 writes flags[v] (0 or 1), so the flags need no clearing beforehand.
__global__ void __launch_bounds__(256) foreground_any_kernel(const uint8_t* rgba, long hw, int* flags) {
  const uchar4* px = reinterpret_cast<const uchar4*>(rgba) + long(blockIdx.x) * hw;
  int any = 0;
  for (long p = threadIdx.x; p < hw && !any; p += blockDim.x) any = px[p].w >= 128;
  any = __syncthreads_or(any);
  if (threadIdx.x == 0) flags[blockIdx.x] = any ? 1 : 0;
}

void foreground_any(const Exec& ex, const uint8_t* rgba, int V, int H, int W, int* flags) {
  if (ex.dry || V == 0) return;
  hipLaunchKernelGGL(foreground_any_kernel, dim3(V), dim3(256), 0, ex.stream, rgba, long(H) * W, flags);
  SPLAT_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------------------
// image 0.25.10 imageops::resize on RGBA8 (sample.rs: vertical_sample, then horizontal_sample):
// pass 1 tmp[y, x] = sum_i w_y[i] * src[first_y + i, x] in f32, taps in order from 0; pass 2
// dst[y, x] = round_half_away(clamp(sum_i w_x[i] * tmp[y, first_x + i], 0, 255)). Products and
// sums are rounded separately, as the crate's `t += p * w` (no contraction), so the device
// reproduces the crate's f32 arithmetic given its weights (computed on the host, preprocess.cpp).
// One thread per output pixel, 4 channels.
#pragma clang fp contract(off)
__global__ void __launch_bounds__(256) resize_rows_kernel(const uint8_t* src, int W, int NH, const int* first,
                                                          const int* count, const int* offset, const float* wts,
                                                          float* tmp) {
  const long id = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= (long)NH * W) return;
  const int y = int(id / W), x = int(id - (long)y * W);
  const int f = first[y], n = count[y];
  const float* w = wts + offset[y];
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
  for (int i = 0; i < n; ++i) {
    const uchar4 px = reinterpret_cast<const uchar4*>(src)[(long)(f + i) * W + x];
    const float wi = w[i];
    a0 = a0 + float(px.x) * wi;
    a1 = a1 + float(px.y) * wi;
    a2 = a2 + float(px.z) * wi;
    a3 = a3 + float(px.w) * wi;
  }
  reinterpret_cast<float4*>(tmp)[id] = make_float4(a0, a1, a2, a3);
}

__device__ inline uint8_t to_u8_nearest(float v) { return uint8_t(roundf(v < 0.f ? 0.f : v > 255.f ? 255.f : v)); }

__global__ void __launch_bounds__(256) resize_cols_kernel(const float* tmp, int W, int NH, int NW, const int* first,
                                                          const int* count, const int* offset, const float* wts,
                                                          uint8_t* dst) {
  const long id = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= (long)NH * NW) return;
  const int y = int(id / NW), x = int(id - (long)y * NW);
  const int f = first[x], n = count[x];
  const float* w = wts + offset[x];
  const float4* row = reinterpret_cast<const float4*>(tmp) + (long)y * W + f;
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
  for (int i = 0; i < n; ++i) {
    const float4 px = row[i];
    const float wi = w[i];
    a0 = a0 + px.x * wi;
    a1 = a1 + px.y * wi;
    a2 = a2 + px.z * wi;
    a3 = a3 + px.w * wi;
  }
  reinterpret_cast<uchar4*>(dst)[id] = make_uchar4(to_u8_nearest(a0), to_u8_nearest(a1), to_u8_nearest(a2), to_u8_nearest(a3));
}
#pragma clang fp contract(on)

void resize_rgba8(const Exec& ex, const uint8_t* src, int W, int H, float* tmp, uint8_t* dst, int NW, int NH,
                  const ResizeTaps& rows, const ResizeTaps& cols) {
  SPLAT_CHECK(W > 0 && H > 0 && NW > 0 && NH > 0, BAD_ARGUMENT, "resize_rgba8 sizes");
  if (ex.dry) return;
  ProfScope ps(ex, "resize_rgba8", 0, double(W) * H * 4 + double(NW) * NH * 4);
  hipLaunchKernelGGL(resize_rows_kernel, dim3(cdiv(long(NH) * W, 256)), dim3(256), 0, ex.stream, src, W, NH, rows.first,
                     rows.count, rows.offset, rows.w, tmp);
  SPLAT_HIP(hipGetLastError());
  hipLaunchKernelGGL(resize_cols_kernel, dim3(cdiv(long(NH) * NW, 256)), dim3(256), 0, ex.stream, tmp, W, NH, NW,
                     cols.first, cols.count, cols.offset, cols.w, dst);
  SPLAT_HIP(hipGetLastError());
}

}  // namespace splat
