// MFMA GEMM with fused prologue (implicit-im2col conv, ReLU-on-load) and epilogue (bias,
// GELU/ReLU, table add, LayerScale, up to two residuals, row remap, transposed-conv scatter).
//
// Both operands are "K-contiguous": A [M, K] (or an implicit im2col of an NHWC map) and
// W [N, K] (PyTorch Linear / conv weight order). A k-tile is 128 bytes of K per row (64 bf16
// or 32 fp32). Each lane feeds the matrix core a 16-byte fragment of one row: lanes 0-31 the
// first 16 bytes of a 32-byte k-step, lanes 32-63 the second; A and W use the same k order,
// so the sum over k is exact whatever order the hardware walks the fragment in.
//   bf16: one v_mfma_f32_32x32x16_bf16 per k-step;
//   fp32: 64-byte k-steps on v_mfma_f32_16x16x4_f32 (it sustains ~145 TFLOP/s on this part,
//   v_mfma_f32_32x32x2_f32 ~120): lane l reads 16 bytes of row l%16 of each 16-row half of a
//   32-row tile, chunk 4 s + l/16 of the step, and product e of a half pair takes float e of
//   those fragments (k-slot l/16 = chunk l/16).
// Accumulator layout per 32x32 tile (f32x16): bf16, lane l, register r -> row 8*(r/4) +
// 4*(l/32) + r%4, column l%32; fp32, registers 4 (2 mi + ni) + r -> row 16 mi + 4*(l/16) + r,
// column 16 ni + l%16.
#include "kernels.h"

#include <algorithm>
#include <type_traits>

namespace splat {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short short2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

template <typename T> struct Mfma;
template <> struct Mfma<bf16> {
  __device__ static inline void mma(f32x16& acc, const uint4& a, const uint4& b) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                  acc, 0, 0, 0);
  }
  // max(x, 0) of bf16 pairs as signed 16-bit integers (one v_pk_max_i16 a dword): negative
  // values, -0 included, have the sign bit set and compare below 0.
  __device__ static inline uint4 relu(uint4 v) {
    uint32_t* w = reinterpret_cast<uint32_t*>(&v);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(short2_t, w[i]), short2_t{0, 0}));
    return v;
  }
};
template <> struct Mfma<f16> {
  __device__ static inline void mma(f32x16& acc, const uint4& a, const uint4& b) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b),
                                                 acc, 0, 0, 0);
  }
  __device__ static inline uint4 relu(uint4 v) { return Mfma<bf16>::relu(v); }  // same sign-bit rule
};
template <> struct Mfma<float> {
  // One 64-byte k-step of a 32x32 tile as 2 x 2 halves of 16 rows / 16 columns: a0, a1 the A
  // fragments of rows 0-15 and 16-31, b0, b1 the W fragments of columns 0-15 and 16-31.
  __device__ static inline void mma2x2(f32x16& acc, const uint4& a0, const uint4& a1, const uint4& b0,
                                       const uint4& b1) {
    f32x4 c0 = acc.s0123, c1 = acc.s4567, c2 = acc.s89ab, c3 = acc.scdef;
    const float* x0 = reinterpret_cast<const float*>(&a0);
    const float* x1 = reinterpret_cast<const float*>(&a1);
    const float* y0 = reinterpret_cast<const float*>(&b0);
    const float* y1 = reinterpret_cast<const float*>(&b1);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      c0 = __builtin_amdgcn_mfma_f32_16x16x4f32(x0[e], y0[e], c0, 0, 0, 0);
      c1 = __builtin_amdgcn_mfma_f32_16x16x4f32(x0[e], y1[e], c1, 0, 0, 0);
      c2 = __builtin_amdgcn_mfma_f32_16x16x4f32(x1[e], y0[e], c2, 0, 0, 0);
      c3 = __builtin_amdgcn_mfma_f32_16x16x4f32(x1[e], y1[e], c3, 0, 0, 0);
    }
    acc.s0123 = c0;
    acc.s4567 = c1;
    acc.s89ab = c2;
    acc.scdef = c3;
  }
  __device__ static inline void mma(f32x16& acc, const uint4& a, const uint4& b) {
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.x), __uint_as_float(b.x), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.y), __uint_as_float(b.y), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.z), __uint_as_float(b.z), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.w), __uint_as_float(b.w), acc, 0, 0, 0);
  }
  __device__ static inline uint4 relu(uint4 v) {  // max(x, 0) as signed integers (v_max_i32)
    uint32_t* w = reinterpret_cast<uint32_t*>(&v);
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = uint32_t(max(int(w[i]), 0));
    return v;
  }
};

// Exact (erf) GELU, x * Phi(x). erfc(z) for z = |x|/sqrt(2) >= 0 follows Abramowitz & Stegun
// 7.1.26: t (a1 + t (a2 + t (a3 + t (a4 + t a5)))) exp(-z^2) with t = 1/(1 + p z), absolute
// error <= 1.5e-7. With h = |x| erfc(z) / 2 (the a_i halved, exp(-z^2) = 2^(x^2 (-log2(e) / 2)))
// the result is max(x, 0) - h for either sign: x - x erfc(z)/2 for x >= 0 and x erfc(z)/2 for
// x < 0, without the cancellation of 1 + erf(x/sqrt(2)). 13 VALU instructions (two of them
// v_rcp and v_exp) where a sign select took 16, against the library erff's 30-40 (the GELU
// epilogue is VALU-bound: 6222x4096 fc1 94.6 -> 77.1 us with the select form, 62.0 us without
// an activation).
__device__ inline float gelu_erf(float x) {
  const float ax = fabsf(x);
  const float t = __builtin_amdgcn_rcpf(fmaf(ax, 0.3275911f * 0.70710678118654752f, 1.f));
  const float p =
      t * (0.127414796f + t * (-0.142248368f + t * (0.7107068705f + t * (-0.7265760135f + t * 0.5307027145f))));
  const float h = p * __builtin_amdgcn_exp2f(x * x * -0.72134752044448170f);
  return fmaf(-ax, h, fmaxf(x, 0.f));
}

// A residual is fp32 when flagged, else stored in the kernel's own dtype T.
template <typename T>
__device__ inline float load_res(const void* p, long i, int f32) {
  if constexpr (sizeof(T) == 4) return reinterpret_cast<const float*>(p)[i];
  else return f32 ? reinterpret_cast<const float*>(p)[i] : u16f<T>(reinterpret_cast<const uint16_t*>(p)[i]);
}

// Output index of element (m, n): row-major with optional row remap, or the transposed-conv
// scatter (n = (dy*s + dx)*Cout + co of input pixel m -> NHWC output pixel).
__device__ inline long out_index(const GemmArgs& p, long m, long n, long row) {
  if (p.store != STORE_CONVT) return row * p.ldc + n;
  const long t = n / p.ct_Cout, co = n - t * p.ct_Cout;
  const long dy = t / p.ct_s, dx = t - dy * p.ct_s;
  const long hw = (long)p.ct_R * p.ct_C;
  const long vv = m / hw, rem = m - vv * hw;
  const long rr = rem / p.ct_C, cc = rem - rr * p.ct_C;
  return ((vv * p.ct_R * p.ct_s + rr * p.ct_s + dy) * ((long)p.ct_C * p.ct_s) + cc * p.ct_s + dx) * p.ct_Cout + co;
}

// 8 consecutive values, fp32 or (f32 false) the 16-bit type T.
template <typename T>
__device__ inline void load8(const void* p, long i, bool f32, float* v) {
  if (f32 || sizeof(T) == 4) {
    const float4 a = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(p) + i);
    const float4 b = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(p) + i + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else if constexpr (sizeof(T) == 2) {
    const uint4 u = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(p) + i);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[2 * k] = u16f<T>(w[k]);
      v[2 * k + 1] = u16f<T>(w[k] >> 16);
    }
  }
}

// Store of 8 consecutive values (16-byte aligned, all inside the array) as fp32 or as T.
template <typename T>
__device__ inline void store8_to(void* base, bool f32, const float* v, long idx) {
  if (f32 || sizeof(T) == 4) {
    float* o = reinterpret_cast<float*>(base) + idx;
    *reinterpret_cast<float4*>(o) = make_float4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<float4*>(o + 4) = make_float4(v[4], v[5], v[6], v[7]);
  } else if constexpr (sizeof(T) == 2) {
    uint4 u;
    u.x = pack2<T>(v[0], v[1]);
    u.y = pack2<T>(v[2], v[3]);
    u.z = pack2<T>(v[4], v[5]);
    u.w = pack2<T>(v[6], v[7]);
    *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(base) + idx) = u;
  }
}
// Store of 8 consecutive output values.
template <typename T>
__device__ inline void store8(const GemmArgs& p, const float* v, long idx) {
  store8_to<T>(p.out, p.out_f32, v, idx);
}

// Epilogue of 8 consecutive columns n..n+7 of row m: bias, activation, table add, LayerScale,
// residuals, post-residual activation, store. `vec`: all of them exist and every operand is
// 16-byte aligned for them.
template <typename T>
__device__ inline void epi8(const GemmArgs& p, float* v, long m, long n, bool vec) {
  const long row = p.rm_P ? (m / p.rm_P) * p.rm_n + p.rm_off + m % p.rm_P : m;
  const bool rf = p.res_f32 || sizeof(T) == 4, rf2 = p.res2_f32 || sizeof(T) == 4;
  if (vec) {
    float t[8];
    if (p.bias) { load8<T>(p.bias, n, true, t); for (int k = 0; k < 8; ++k) v[k] += t[k]; }
    if (p.act == ACT_RELU) for (int k = 0; k < 8; ++k) v[k] = fmaxf(v[k], 0.f);
    else if (p.act == ACT_GELU) for (int k = 0; k < 8; ++k) v[k] = gelu_erf(v[k]);
    if (p.addtab) { load8<T>(p.addtab, (m % p.addtab_period) * p.N + n, true, t); for (int k = 0; k < 8; ++k) v[k] += t[k]; }
    if (p.gamma) { load8<T>(p.gamma, n, true, t); for (int k = 0; k < 8; ++k) v[k] *= t[k]; }
    if (p.res) { load8<T>(p.res, row * p.ldres + n, rf, t); for (int k = 0; k < 8; ++k) v[k] += t[k]; }
    if (p.res2) { load8<T>(p.res2, row * p.ldres2 + n, rf2, t); for (int k = 0; k < 8; ++k) v[k] += t[k]; }
    if (p.act_post == ACT_GELU) for (int k = 0; k < 8; ++k) v[k] = gelu_erf(v[k]);
    else if (p.act_post == ACT_RELU) for (int k = 0; k < 8; ++k) v[k] = fmaxf(v[k], 0.f);
    store8<T>(p, v, out_index(p, m, n, row));
    return;
  }
  for (int k = 0; k < 8; ++k) {
    const long nn = n + k;
    if (nn >= p.N) break;
    float x = v[k] + (p.bias ? p.bias[nn] : 0.f);
    if (p.act == ACT_RELU) x = fmaxf(x, 0.f);
    else if (p.act == ACT_GELU) x = gelu_erf(x);
    if (p.addtab) x += p.addtab[(m % p.addtab_period) * p.N + nn];
    if (p.gamma) x *= p.gamma[nn];
    if (p.res) x += load_res<T>(p.res, row * p.ldres + nn, p.res_f32);
    if (p.res2) x += load_res<T>(p.res2, row * p.ldres2 + nn, p.res2_f32);
    if (p.act_post == ACT_GELU) x = gelu_erf(x);
    else if (p.act_post == ACT_RELU) x = fmaxf(x, 0.f);
    const long idx = out_index(p, m, nn, row);
    if (p.out_f32) reinterpret_cast<float*>(p.out)[idx] = x;
    else reinterpret_cast<T*>(p.out)[idx] = from_f<T>(x);
  }
}

// Epilogue through LDS: each wave stages one 32-row slab of its accumulators at a time
// (from the 32x32 accumulator layout: lane l, register r -> row 8*(r/4) + 4*(l/32) + r%4,
// column l%32 of each 32x32 tile), then every lane finishes runs of 8 consecutive columns.
// Three compile-time variants keep the code that a launch runs small (the unrolled slabs
// multiply every optional feature, and instruction fetch, not memory, then bounds the
// epilogue):
//   EPI_BIAS  out = act(acc + bias)                          row-major, 16-byte runs
//   EPI_RES   out = act(acc + bias) * gamma + res (+ res2)   row-major, 16-byte runs
//   EPI_FULL  every feature (table add, row remap, second residual, transposed-conv
//             scatter, unaligned or ragged runs) through epi8.
// In the first two a lane always owns the same column run (RUNS divides 64), so bias and
// LayerScale are loaded once, and the residuals of CH runs are requested before the first of
// those runs is stored. `slab` is this wave's LDS region of 32 x slab_ld(TN) floats; the
// block must be past its last read of the main-loop LDS.
// EPI_PART: split-K slice, the raw fp32 sums go to the partial buffer; a reduce kernel adds
// the slices and applies the full epilogue.
// EPI_LN: EPI_BIAS with the folded LayerNorm of the A rows (GemmArgs::ln_in): rstd * (acc -
// mean * c1), with (rstd, -rstd * mean) of each tile row reduced from its partial statistics by
// one thread at the kernel's start (the loads go out ahead of the first operand tiles) and kept
// in LDS for the epilogue. EPI_RESLN: EPI_RES that also emits the statistics of its output rows
// (GemmArgs::ln_out) and their copy in the GEMM's dtype: each 4-lane group of a row sums its 32
// columns (DPP), the sums meet in LDS past the slabs, and after the last slab the block writes
// one (sum, sum of squares) pair per row and column group.
enum EpiKind { EPI_BIAS = 0, EPI_RES = 1, EPI_FULL = 2, EPI_PART = 3, EPI_HEAD = 4, EPI_LN = 5, EPI_RESLN = 6 };

// Sum over the G consecutive lanes of a group (G = 4, 8 or 16, groups aligned), left in every
// lane of the group: quad swaps, then the half-row and row mirrors.
template <int G> __device__ __forceinline__ float group_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xf, 0xf, true));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xf, 0xf, true));
  if (G >= 8) v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xf, 0xf, true));
  if (G >= 16) v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xf, 0xf, true));
  return v;
}

constexpr int slab_ld(int tn) { return tn * 32 + 4; }  // +4 floats: conflict-free 16-byte row reads

// A __shared__ float array of N elements, or none (nullptr) when N is 0: a kernel whose operand
// ring fills the LDS declares nothing else.
template <int N> struct LdsFloats {
  __device__ static float* get() {
    __shared__ __attribute__((aligned(16))) float a[N];
    return a;
  }
};
template <> struct LdsFloats<0> {
  __device__ static float* get() { return nullptr; }
};


template <int TM, int TN, bool L16>
__device__ __forceinline__ void stage_slab(const f32x16 (&acc)[TM][TN], int i, float* slab, int lane) {
  constexpr int LD = slab_ld(TN);
  if constexpr (L16) {  // fp32: 16x16 halves, registers 4 (2 mi + ni) + r
    const int q = lane >> 4, l16 = lane & 15;
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        slab[(16 * (r >> 3) + 4 * q + (r & 3)) * LD + j * 32 + 16 * ((r >> 2) & 1) + l16] = acc[i][j][r];
  } else {
    const int g = lane >> 5, l32 = lane & 31;
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) slab[(8 * (r >> 2) + 4 * g + (r & 3)) * LD + j * 32 + l32] = acc[i][j][r];
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ void slab_done() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ void read8(const float* q, float* v) {
  const float4 a = *reinterpret_cast<const float4*>(q);
  const float4 b = *reinterpret_cast<const float4*>(q + 4);
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// qk-norm + RoPE (GemmArgs::qk_dim) of a wave's column runs n..n+7 in CH rows (q or k columns,
// heads 64-column aligned). Channel c0 = n % 64. The head's statistics: with RUNS >= 8 lanes a
// row (waves 64+ columns wide) the 8 lanes of a head reduce them by DPP; with RUNS = 4 (32-column
// waves) each half-head's (sum, sum of squares) meets the other half's in LDS (`xch`, two pairs
// per tile row) across a block barrier. The RoPE partner of channel c (c +- 16 in its 32-channel
// half) is in lane ^ 2 (quad_perm [2,3,0,1]). Every lane of the block calls it, also for v
// columns (`qk` false), so that the barrier is uniform.
template <int RUNS, int CH>
__device__ inline void qk_norm_rope(const GemmArgs& p, float (&v)[CH][8], const long (&m)[CH], long n, int lane,
                                    bool qk, float* xch, const int (&xrow)[CH]) {
  const int c0 = int(n % 64);
  const bool isk = n >= p.qk_dim;
  const float* w = isk ? p.kw : p.qw;
  const float* b = isk ? p.kb : p.qb;
  if (p.qw) {  // LayerNorm over each head's 64 channels (eps 1e-5, vit_block.rs:17)
    float mean[CH], rstd[CH];
    if constexpr (RUNS >= 8) {
#pragma unroll
      for (int t = 0; t < CH; ++t) {
        float s = 0.f;
#pragma unroll
        for (int k = 0; k < 8; ++k) s += v[t][k];
        mean[t] = group_sum<8>(s) * (1.f / 64.f);
        float q = 0.f;
#pragma unroll
        for (int k = 0; k < 8; ++k) q = fmaf(v[t][k] - mean[t], v[t][k] - mean[t], q);
        rstd[t] = rsqrtf(group_sum<8>(q) * (1.f / 64.f) + 1e-5f);
      }
    } else {
      const int half = c0 >> 5;
#pragma unroll
      for (int t = 0; t < CH; ++t) {
        float s = 0.f, q = 0.f;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          s += v[t][k];
          q = fmaf(v[t][k], v[t][k], q);
        }
        s = group_sum<4>(s);
        q = group_sum<4>(q);
        if ((lane & 3) == 0 && qk) {
          xch[(xrow[t] * 2 + half) * 2] = s;
          xch[(xrow[t] * 2 + half) * 2 + 1] = q;
        }
      }
      __syncthreads();
#pragma unroll
      for (int t = 0; t < CH; ++t) {
        const float* e = xch + xrow[t] * 4;
        const float s = e[0] + e[2], q = e[1] + e[3];
        mean[t] = s * (1.f / 64.f);
        rstd[t] = rsqrtf(fmaxf(q * (1.f / 64.f) - mean[t] * mean[t], 0.f) + 1e-5f);
      }
      __syncthreads();  // the exchange area is reused by the next slab
    }
    if (qk) {
#pragma unroll
      for (int t = 0; t < CH; ++t)
#pragma unroll
        for (int k = 0; k < 8; ++k) v[t][k] = (v[t][k] - mean[t]) * rstd[t] * w[c0 + k] + b[c0 + k];
    }
  }
  if (p.rope_cs && qk) {
    const bool first = (c0 & 16) == 0;  // channel c < 16 of its half: pairs with c + 16
#pragma unroll
    for (int t = 0; t < CH; ++t) {
      const long tok = m[t] % p.rope_n;
      int pr = 0, pc = 0;
      if (tok > 0) {
        if (p.rope_across) pr = pc = 1;
        else {
          pr = int((tok - 1) / p.rope_cols) + 1;
          pc = int((tok - 1) % p.rope_cols) + 1;
        }
      }
      const int pos = c0 >= 32 ? pc : pr;  // channels 32-63 rotate by the column position
      const float* cs = p.rope_cs + pos * 16 + (c0 & 8);
      const float* sn = p.rope_cs + (p.rope_npos + pos) * 16 + (c0 & 8);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float pv = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v[t][k]), 0x4E, 0xf, 0xf, true));
        v[t][k] = first ? v[t][k] * cs[k] - pv * sn[k] : v[t][k] * cs[k] + pv * sn[k];
      }
    }
  }
}

// `lnab` (EPI_LN): (rstd, -rstd * mean) of this wave's rows in LDS; `xch` (EPI_LN with
// qk_dim): the block's qk-norm exchange area, xrow0 this wave's first tile row. `lnp`
// (EPI_RESLN): this wave's corner of the LDS array of 32-column sums, lnp_ld a row.
template <typename T, int TM, int TN, int EPI, bool L16 = false>
__device__ __forceinline__ void epilogue(const GemmArgs& p, f32x16 (&acc)[TM][TN], long wrow0, long wcol0, float* slab,
                                         int lane, bool vec, float* part = nullptr, const float* lnab = nullptr,
                                         float* lnp = nullptr, int lnp_ld = 0, float* xch = nullptr, int xrow0 = 0) {
  constexpr int COLS = TN * 32, LD = slab_ld(TN), RUNS = COLS / 8;
  if constexpr (EPI == EPI_PART) {
    // rows of 8 columns: n < N implies n + 8 <= ldp (ldp is N rounded up to 8)
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      stage_slab<TM, TN, L16>(acc, i, slab, lane);
      for (int q = lane; q < 32 * RUNS; q += 64) {
        const int rr = q / RUNS, cc = (q - rr * RUNS) * 8;
        const long m = wrow0 + i * 32 + rr, n = wcol0 + cc;
        if (m < p.M && n < p.N) {
          float* dst = part + m * p.ldp + n;
          *reinterpret_cast<float4*>(dst) = *reinterpret_cast<const float4*>(slab + rr * LD + cc);
          *reinterpret_cast<float4*>(dst + 4) = *reinterpret_cast<const float4*>(slab + rr * LD + cc + 4);
        }
      }
      slab_done();
    }
  } else if constexpr (EPI == EPI_FULL) {
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      stage_slab<TM, TN, L16>(acc, i, slab, lane);
      for (int q = lane; q < 32 * RUNS; q += 64) {
        const int rr = q / RUNS, cc = (q - rr * RUNS) * 8;
        const long m = wrow0 + i * 32 + rr, n = wcol0 + cc;
        if (m < p.M && n < p.N) {
          float v[8];
          read8(slab + rr * LD + cc, v);
          epi8<T>(p, v, m, n, vec && n + 8 <= p.N);
        }
      }
      slab_done();
    }
  } else {
    constexpr bool RES = EPI == EPI_RES || EPI == EPI_RESLN;
    constexpr int IT = 32 * RUNS / 64;   // runs per lane per slab
    constexpr int CH = IT < 4 ? IT : 4;  // runs whose residual loads are in flight together
    static_assert(64 % RUNS == 0 && IT % CH == 0, "run layout");
    const int cc = (lane % RUNS) * 8, rsub = lane / RUNS;
    const long n = wcol0 + cc;
    const bool nok = n < p.N;  // the host guarantees that a run starting inside the output lies in it
    float cb[8], cg[8], c1[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) { cb[k] = 0.f; cg[k] = 1.f; c1[k] = 0.f; }
    if (nok && p.bias) load8<T>(p.bias, n, true, cb);
    if (RES && nok && p.gamma) load8<T>(p.gamma, n, true, cg);
    if (EPI == EPI_LN && nok) load8<T>(p.ln_c1, n, true, c1);
    const bool rf = p.res_f32 || sizeof(T) == 4, rf2 = p.res2_f32 || sizeof(T) == 4;
    // The residual runs of slab i + 1 are requested while slab i is staged and stored, so that
    // only the first slab's wait is exposed.
    float rvn[IT][8];
    auto load_res = [&](int i) {
#pragma unroll
      for (int t = 0; t < IT; ++t) {
        const long m = wrow0 + i * 32 + rsub + t * (64 / RUNS);
        if (RES && p.res && nok && m < p.M) load8<T>(p.res, m * p.ldres + n, rf, rvn[t]);
        else if (RES) {
#pragma unroll
          for (int k = 0; k < 8; ++k) rvn[t][k] = 0.f;
        }
      }
    };
    load_res(0);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      float rvs[IT][8];
#pragma unroll
      for (int t = 0; t < IT; ++t)
#pragma unroll
        for (int k = 0; k < 8; ++k) rvs[t][k] = rvn[t][k];
      if (i + 1 < TM) load_res(i + 1);
      float la[IT], lb[IT];  // folded LayerNorm of this lane's rows
      if constexpr (EPI == EPI_LN) {
#pragma unroll
        for (int t = 0; t < IT; ++t) {
          const float2 ab = *reinterpret_cast<const float2*>(lnab + (i * 32 + rsub + t * (64 / RUNS)) * 2);
          la[t] = ab.x;
          lb[t] = ab.y;
        }
      }
      stage_slab<TM, TN, L16>(acc, i, slab, lane);
#pragma unroll
      for (int t0 = 0; t0 < IT; t0 += CH) {
        float v[CH][8], rv[CH][8];
#pragma unroll
        for (int t = 0; t < CH; ++t) {
          const int rr = rsub + (t0 + t) * (64 / RUNS);
          read8(slab + rr * LD + cc, v[t]);
          if (RES && p.res) {
#pragma unroll
            for (int k = 0; k < 8; ++k) rv[t][k] = rvs[t0 + t][k];
          }
        }
        if (RES && p.res2) {  // second residual (the DPT residual units' skip input)
#pragma unroll
          for (int t = 0; t < CH; ++t) {
            const long m = wrow0 + i * 32 + rsub + (t0 + t) * (64 / RUNS);
            float r2[8];
            if (nok && m < p.M) {
              load8<T>(p.res2, m * p.ldres2 + n, rf2, r2);
#pragma unroll
              for (int k = 0; k < 8; ++k) rv[t][k] += r2[k];
            }
          }
        }
#pragma unroll
        for (int t = 0; t < CH; ++t) {
          float* x = v[t];
          if constexpr (EPI == EPI_LN) {
#pragma unroll
            for (int k = 0; k < 8; ++k) x[k] = fmaf(la[t0 + t], x[k], fmaf(lb[t0 + t], c1[k], cb[k]));
          } else {
#pragma unroll
            for (int k = 0; k < 8; ++k) x[k] += cb[k];
          }
          if (p.act == ACT_RELU) {
#pragma unroll
            for (int k = 0; k < 8; ++k) x[k] = fmaxf(x[k], 0.f);
          } else if (p.act == ACT_GELU) {
#pragma unroll
            for (int k = 0; k < 8; ++k) x[k] = gelu_erf(x[k]);
          }
        }
        if constexpr (EPI == EPI_LN) {
          if (p.qk_dim) {  // block-uniform (a barrier inside for 32-column waves)
            static_assert(EPI != EPI_LN || CH == IT, "qk-norm: a slab's rows in one chunk");
            long mm[CH];
            int xr[CH];
#pragma unroll
            for (int t = 0; t < CH; ++t) {
              xr[t] = xrow0 + i * 32 + rsub + (t0 + t) * (64 / RUNS);
              mm[t] = wrow0 + i * 32 + rsub + (t0 + t) * (64 / RUNS);
            }
            qk_norm_rope<RUNS, CH>(p, v, mm, n, lane, wcol0 < 2 * p.qk_dim, xch, xr);
          }
          if (n < p.q_cols) {
#pragma unroll
            for (int t = 0; t < CH; ++t)
#pragma unroll
              for (int k = 0; k < 8; ++k) v[t][k] *= p.q_scale;
          }
        }
        if constexpr (EPI == EPI_LN) {
          if (p.glu) {
            // SwiGLU: even runs hold x1 channels 8j..8j+7, the next lane's run the matching x2
            // ones; the even lane stores silu(x1) * x2 at output column n / 2
#pragma unroll
            for (int t = 0; t < CH; ++t) {
              const int rr = rsub + (t0 + t) * (64 / RUNS);
              const long m = wrow0 + i * 32 + rr;
              float y[8];
#pragma unroll
              for (int k = 0; k < 8; ++k) {
                const float x2 = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v[t][k]), 0xB1, 0xf, 0xf, true));
                y[k] = v[t][k] / (1.f + __expf(-v[t][k])) * x2;
              }
              if (nok && m < p.M && (lane & 1) == 0) store8<T>(p, y, m * p.ldc + n / 2);
            }
            continue;
          }
        }
#pragma unroll
        for (int t = 0; t < CH; ++t) {
          const int rr = rsub + (t0 + t) * (64 / RUNS);
          const long m = wrow0 + i * 32 + rr;
          float* x = v[t];
          if (RES) {
#pragma unroll
            for (int k = 0; k < 8; ++k) x[k] *= cg[k];
            if (p.res) {
#pragma unroll
              for (int k = 0; k < 8; ++k) x[k] += rv[t][k];
            }
          }
          const bool ok = nok && m < p.M;
          if constexpr (EPI == EPI_RESLN) {
            float s = 0.f, q = 0.f;
            if (ok) {
#pragma unroll
              for (int k = 0; k < 8; ++k) {
                s += x[k];
                q = fmaf(x[k], x[k], q);
              }
            }
            s = group_sum<4>(s);  // the 4 lanes of one 32-column group
            q = group_sum<4>(q);
            if ((lane & 3) == 0) {
              float* dst = lnp + ((i * 32 + rr) * lnp_ld + cc / 32) * 2;
              dst[0] = s;
              dst[1] = q;
            }
            if (ok && p.ln_copy) store8_to<T>(p.ln_copy, false, x, m * p.ldc + n);  // the GEMM's dtype
          }
          if (ok) store8<T>(p, x, m * p.ldc + n);
        }
      }
      slab_done();
    }
  }
}

// EPI_HEAD: the MapAnything output head (mapanything-rs/src/dpt.rs:196-198 conv2.2 and
// model.rs:148-172 dense_output) on the tile's pixels, which hold all N = 128 channels. Each
// lane takes 8 channels of a slab row: h = bf16(relu(acc + bias)), 6 partial dot products with
// the 1x1 weights, summed over the row's lanes by DPP; the waves' partials per row meet in LDS
// after the slabs (the ring is free by then), and one thread per pixel finishes the outputs.
template <typename T, int BM, int BN, int WM, int WN, int TM, int TN, bool L16 = false>
__device__ __forceinline__ void head_epilogue(const GemmArgs& p, f32x16 (&acc)[TM][TN], long m0, int wm, int wn,
                                              float* smemf, int wave, int lane, int tid) {
  constexpr int NW = WM * WN, COLS = TN * 32, LD = slab_ld(TN), RUNS = COLS / 8, RPP = 64 / RUNS;
  static_assert(BN == 128 && (RUNS == 4 || RUNS == 8), "head epilogue: all 128 channels, 4 or 8 lanes a row");
  float* slab = smemf + wave * 32 * LD;
  float* part = smemf + NW * 32 * LD;  // [BM][WN][6]
  const int cc = (lane % RUNS) * 8, rsub = lane / RUNS;
  const int c0 = wn * (BN / WN) + cc;
  float wt[6][8], cb[8];
#pragma unroll
  for (int o = 0; o < 6; ++o)
#pragma unroll
    for (int k = 0; k < 8; ++k) wt[o][k] = p.hw3[o * 128 + c0 + k];
#pragma unroll
  for (int k = 0; k < 8; ++k) cb[k] = p.bias[c0 + k];
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    stage_slab<TM, TN, L16>(acc, i, slab, lane);
#pragma unroll
    for (int t = 0; t < 32 / RPP; ++t) {
      const int rr = rsub + t * RPP;
      float v[8];
      read8(slab + rr * LD + cc, v);
      float s[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float h = to_f<T>(from_f<T>(fmaxf(v[k] + cb[k], 0.f)));
#pragma unroll
        for (int o = 0; o < 6; ++o) s[o] = fmaf(wt[o][k], h, s[o]);
      }
#pragma unroll
      for (int o = 0; o < 6; ++o) {
        s[o] += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s[o]), 0xB1, 0xf, 0xf, true));
        s[o] += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s[o]), 0x4E, 0xf, 0xf, true));
        if (RUNS == 8) s[o] += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s[o]), 0x141, 0xf, 0xf, true));
      }
      if (lane % RUNS == 0) {
        float* dst = part + ((wm * (BM / WM) + i * 32 + rr) * WN + wn) * 6;
#pragma unroll
        for (int o = 0; o < 6; ++o) dst[o] = s[o];
      }
    }
    slab_done();
  }
  __syncthreads();
  const float sc = p.hscale ? *p.hscale : 1.f;
  for (int r = tid; r < BM; r += NW * 64) {
    const long px = m0 + r;
    if (px >= p.M) continue;
    float raw[6];
#pragma unroll
    for (int o = 0; o < 6; ++o) {
      float acc6 = p.hb3[o];
#pragma unroll
      for (int w = 0; w < WN; ++w) acc6 += part[(r * WN + w) * 6 + o];
      raw[o] = acc6;
    }
    const long v = px / p.hhw, q = px - v * p.hhw;
    if (p.ho0) {
#pragma unroll
      for (int o = 0; o < 6; ++o) p.ho0[(v * 6 + o) * p.hhw + q] = raw[o];
    }
    // mapanything-rs/src/model.rs:155-168
    const float nrm = fmaxf(sqrtf(raw[0] * raw[0] + raw[1] * raw[1] + raw[2] * raw[2]), 1e-8f);
    const float depth = expf(raw[3]) * sc;
    if (p.ho1) {
#pragma unroll
      for (int j = 0; j < 3; ++j) p.ho1[px * 3 + j] = raw[j] / nrm * depth;
    }
    if (p.ho2) p.ho2[px] = 1.f + expf(raw[4]);
    if (p.ho3) p.ho3[px] = raw[5] > 0.f ? 1 : 0;
  }
}

// Which epilogue variant a launch needs (host side; `a.epi_vec` already set).
inline int epi_kind(const GemmArgs& a) {
  if (a.hw3) return EPI_HEAD;
  if (!a.epi_vec || a.rm_P || a.store != STORE_ROWS || a.addtab || a.act_post || (a.res2 && !a.res)) return EPI_FULL;
  if (a.ln_in) return (a.res || a.gamma || a.res2) ? EPI_FULL : EPI_LN;  // EPI_FULL: refused by gemm()
  if (a.res || a.gamma) return (a.ln_out && !a.res2) ? EPI_RESLN : EPI_RES;
  return EPI_BIAS;
}

// Whether the 8-column vector path is valid for every run of a launch (host side).
inline bool epi_vec_ok(const GemmArgs& a, size_t es) {
  auto al = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
  const size_t oes = a.out_f32 ? 4 : es;
  bool ok = a.N % 8 == 0 && al(a.out) && (a.bias == nullptr || al(a.bias)) && (a.gamma == nullptr || al(a.gamma)) &&
            (a.addtab == nullptr || al(a.addtab)) && (a.ln_c1 == nullptr || al(a.ln_c1)) &&
            (a.ln_copy == nullptr || al(a.ln_copy));
  if (a.store == STORE_CONVT) ok = ok && a.ct_Cout % 8 == 0;
  else ok = ok && (a.ldc * oes) % 16 == 0;
  if (a.res) ok = ok && al(a.res) && (a.ldres * (a.res_f32 ? 4 : es)) % 16 == 0;
  if (a.res2) ok = ok && al(a.res2) && (a.ldres2 * (a.res2_f32 ? 4 : es)) % 16 == 0;
  if (a.ln_copy) ok = ok && (a.ldc * es) % 16 == 0;
  return ok;
}

constexpr int LDS_ROW = 144;  // bytes per tile row: 128 bytes of K + 16 bytes against bank conflicts

template <typename T, int BM, int BN, int WM, int WN, int AMODE>
__global__ void __launch_bounds__(256) gemm_kernel(const GemmArgs p) {
  constexpr int KE = 16 / sizeof(T);        // elements per 16-byte chunk
  constexpr int BK = 8 * KE;                // elements per k-tile
  constexpr int TM = BM / WM / 32, TN = BN / WN / 32;
  constexpr int ACH = BM / 32, BCH = BN / 32;  // 16-byte chunks per thread per tile
  __shared__ __attribute__((aligned(16))) char smem[2 * (BM + BN) * LDS_ROW];
  static_assert(2 * (BM + BN) * LDS_ROW >= 4 * 32 * slab_ld(TN) * 4, "epilogue slabs reuse the tiles");

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int g = lane >> 5, l32 = lane & 31;
  const long m0 = (long)blockIdx.x * BM, n0 = (long)blockIdx.y * BN;
  const int kc = tid & 7, r0 = tid >> 3;

  // ---- per-thread A row state
  const T* arow[ACH];
  int av[ACH], aiy[ACH], aix[ACH];
  bool aok[ACH];
#pragma unroll
  for (int i = 0; i < ACH; ++i) {
    long m = m0 + r0 + 32 * i;
    aok[i] = m < p.M;
    long mm = aok[i] ? m : 0;
    if (AMODE == A_ROWS) {
      arow[i] = reinterpret_cast<const T*>(p.A) + mm * p.lda;
    } else {
      int hw = p.Ho * p.Wo;
      int v = int(mm / hw), rem = int(mm - (long)v * hw);
      int oy = rem / p.Wo, ox = rem - oy * p.Wo;
      av[i] = v;
      aiy[i] = oy * p.stride - p.pad;
      aix[i] = ox * p.stride - p.pad;
      arow[i] = reinterpret_cast<const T*>(p.A) + (long)v * p.Hi * p.Wi * p.Cin;
    }
  }
  const T* brow[BCH];
  bool bok[BCH];
#pragma unroll
  for (int i = 0; i < BCH; ++i) {
    long n = n0 + r0 + 32 * i;
    bok[i] = n < p.N;
    brow[i] = reinterpret_cast<const T*>(p.W) + (bok[i] ? n : 0) * p.ldw;
  }

  uint4 ra[ACH], rb[BCH];
  auto gload = [&](int kt) {
    const int k = kt * BK + kc * KE;
    const bool kin = k < p.K;
    if (AMODE == A_ROWS) {
#pragma unroll
      for (int i = 0; i < ACH; ++i)
        ra[i] = (aok[i] && kin) ? *reinterpret_cast<const uint4*>(arow[i] + k) : make_uint4(0, 0, 0, 0);
    } else {
      const int tap = k / p.Cin, ci = k - tap * p.Cin;
      const int ky = tap / p.ks, kx = tap - ky * p.ks;
#pragma unroll
      for (int i = 0; i < ACH; ++i) {
        const int iy = aiy[i] + ky, ix = aix[i] + kx;
        const bool ok = aok[i] && kin && iy >= 0 && iy < p.Hi && ix >= 0 && ix < p.Wi;
        ra[i] = ok ? *reinterpret_cast<const uint4*>(arow[i] + ((long)iy * p.Wi + ix) * p.Cin + ci)
                   : make_uint4(0, 0, 0, 0);
      }
    }
    if (p.relu_in) {
#pragma unroll
      for (int i = 0; i < ACH; ++i) ra[i] = Mfma<T>::relu(ra[i]);
    }
#pragma unroll
    for (int i = 0; i < BCH; ++i)
      rb[i] = bok[i] ? *reinterpret_cast<const uint4*>(brow[i] + kt * BK + kc * KE) : make_uint4(0, 0, 0, 0);
  };
  auto sstore = [&](int buf) {
    char* base = smem + buf * (BM + BN) * LDS_ROW;
#pragma unroll
    for (int i = 0; i < ACH; ++i) *reinterpret_cast<uint4*>(base + (r0 + 32 * i) * LDS_ROW + kc * 16) = ra[i];
#pragma unroll
    for (int i = 0; i < BCH; ++i)
      *reinterpret_cast<uint4*>(base + (BM + r0 + 32 * i) * LDS_ROW + kc * 16) = rb[i];
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int nk = (p.K + BK - 1) / BK;
  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) gload(kt + 1);
    const char* base = smem + buf * (BM + BN) * LDS_ROW;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      uint4 fa[TM], fb[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        fa[i] = *reinterpret_cast<const uint4*>(base + (wm * (BM / WM) + i * 32 + l32) * LDS_ROW + (2 * s + g) * 16);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        fb[j] = *reinterpret_cast<const uint4*>(base + (BM + wn * (BN / WN) + j * 32 + l32) * LDS_ROW +
                                                (2 * s + g) * 16);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) Mfma<T>::mma(acc[i][j], fa[i], fb[j]);
    }
    if (kt + 1 < nk) sstore(buf ^ 1);
    __syncthreads();
  }

  float* slab = reinterpret_cast<float*>(smem) + wave * 32 * slab_ld(TN);
  epilogue<T, TM, TN, EPI_FULL>(p, acc, m0 + wm * (BM / WM), n0 + wn * (BN / WN), slab, lane, p.epi_vec);
}

// ---------------------------------------------------------------------------------------
// bf16 main path. Operand tiles stream from global memory straight into LDS through a
// STAGES-deep ring (buffer_load_dwordx4 ... lds: 16 bytes per lane, one wave instruction fills
// 1 KB = 8 tile rows of 128 bytes at BK=64), so no registers stage them, and rows or K-chunks
// outside the operands read as zero through the buffer descriptor's range check (offset
// 0x80000000). Chunk c (16 bytes) of tile row r sits in slot c ^ ((r >> 1) & 7): the 16-lane
// phases of the fragment reads (16 consecutive rows, one chunk) then touch 16 distinct 4-bank
// groups. The loads are inline asm so that the compiler adds no waits of its own; the pipeline
// waits with explicit vmcnt counts and one barrier per k-tile, placed before the tile's last
// k-step so that the first fragments of the next tile are read while that step's MFMAs run.

typedef int int32x4_t __attribute__((ext_vector_type(4)));

__device__ inline int32x4_t make_rsrc(const void* p, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  int32x4_t r;
  r[0] = __builtin_amdgcn_readfirstlane(int(uint32_t(a)));
  r[1] = __builtin_amdgcn_readfirstlane(int(uint32_t(a >> 32)));  // stride 0
  r[2] = __builtin_amdgcn_readfirstlane(int(bytes));
  r[3] = 0x00020000;  // raw buffer, 32-bit data format (gfx9 family)
  return r;
}

typedef const __attribute__((address_space(3))) char* lds_cptr;

__device__ inline uint32_t lds_addr(const void* p) {
  return uint32_t(reinterpret_cast<uintptr_t>((lds_cptr)p));  // generic -> LDS address space cast
}

// 16 bytes per lane from rsrc at voffset + soffset into LDS at lds + 16 * lane. A voffset of
// OOB (or any voffset past the buffer) reads zeros, whatever soffset holds: every valid
// voffset + soffset stays inside the buffer, so the range check of either form (with or
// without soffset) gives the same result.
__device__ inline void load_to_lds(const int32x4_t& rsrc, uint32_t voffset, uint32_t soffset, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(__builtin_amdgcn_readfirstlane(int(lds))),
               "v"(voffset), "s"(rsrc), "s"(__builtin_amdgcn_readfirstlane(int(soffset)))
               : "memory");  // m0 is set here and used by nothing else in these kernels
}

template <int N> __device__ inline void wait_vmcnt() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }

constexpr uint32_t OOB = 0x80000000u;

// Kernel-side A mode of a convolution whose Cin is a multiple of the k-tile and whose filter has
// at most 32 taps (chosen by the launcher; callers pass A_CONV): each k-tile lies in one tap.
constexpr int A_CONV_TAP = 2;

// T = bf16 (one v_mfma_f32_32x32x16_bf16 per k-step) or float (four v_mfma_f32_32x32x2f32):
// a k-step is 32 bytes of K per row either way, so the tiles, loads and swizzles are the same
// byte for byte; BK counts elements (128-byte rows: 64 bf16 or 32 fp32).
// MINB: blocks per CU the register allocation must allow (2 for a tile whose LDS ring lets two
// blocks share a CU).
// AR: ring stages of the A tiles (STAGES those of W). AR = 3 with two W stages (the 256x256 tile,
// exactly the 160 KB of LDS): the loads of A tile kt+2 stream during tile kt, so the load path
// does not drain at every barrier; only the W half is issued after it.
template <typename T, int BM, int BN, int WM, int WN, int STAGES, int BK, int AMODE, bool RELU, int EPI, int MINB,
          int AR = STAGES>
__global__ void __launch_bounds__(WM * WN * 64, MINB) gemm_mfma_kernel(const GemmArgs p, int tiles_m, int tiles_n) {
  constexpr int TM = BM / WM / 32, TN = BN / WN / 32, NW = WM * WN;
  constexpr int ES = sizeof(T), KE = 16 / ES;  // bytes per element, elements per 16-byte chunk
  constexpr int MPI = ES == 4 ? 16 : 1;        // MFMA instructions per tile pair and k-step
  // A tile row holds BK elements = RB bytes = CPR 16-byte chunks; one load instruction of a
  // wave fills RPI rows (1 KiB). Chunk c of row r sits in slot c ^ ((r >> SH) & (CPR - 1)), which
  // keeps the 16 lanes of every ds_read_b128 phase on distinct banks.
  constexpr int RB = BK * ES, CPR = RB / 16, RPI = 64 / CPR, SH = CPR == 8 ? 1 : 2;
  static_assert(RB == 128 || RB == 64, "k-tile");
  // fp32: 64-byte k-steps on 16x16x4 products, two fragments (16-row halves) per 32-row tile
  constexpr bool L16 = ES == 4;
  static_assert(!L16 || RB == 128, "fp32 k-tiles are 128 bytes");
  constexpr int KS = L16 ? RB / 64 : RB / 32;
  constexpr int FH = L16 ? 2 : 1;  // fragments per 32-row tile per k-step
  constexpr int AL = BM / (NW * RPI), BL = BN / (NW * RPI);  // load instructions per wave per k-tile
  constexpr int LPT = AL + BL;
  static_assert(AL * NW * RPI == BM && BL * NW * RPI == BN, "tile rows split evenly over the waves' loads");
  static_assert(((NW * RPI) >> SH) % CPR == 0, "a load's swizzle slot is the same for every instruction");
  constexpr int STAGE = (BM + BN) * RB;
  constexpr bool SPLITR = AR != STAGES;
  static_assert(!SPLITR || (STAGES == 2 && AR == 3), "split ring: three A stages, two W stages");
  constexpr int RING = SPLITR ? AR * BM * RB + STAGES * BN * RB : STAGES * STAGE;
  static_assert((STAGES - 1) * LPT <= 63, "vmcnt range");
  static_assert(RING >= NW * 32 * slab_ld(TN) * 4, "epilogue slabs reuse the ring");
  static_assert(EPI != EPI_LN || NW * 64 >= BM, "folded LayerNorm: a thread per tile row");
  // EPI_LN past the slabs: the qk-norm exchange, then (split ring) the rows' (rstd, -rstd * mean)
  constexpr int XCH = (WN + 1) / 2 * BM * 4;
  static_assert(EPI != EPI_LN || RING >= (NW * 32 * slab_ld(TN) + XCH + (SPLITR ? 2 * BM : 0)) * 4,
                "qk-norm exchange past the epilogue slabs");
  static_assert(EPI != EPI_RESLN || RING >= (NW * 32 * slab_ld(TN) + BM * (BN / 32) * 2) * 4,
                "row statistics: the 32-column sums past the epilogue slabs");
  __shared__ __attribute__((aligned(1024))) char smem[RING];
  // (rstd, -rstd * mean) a row (EPI_LN): its own array, or with the split ring in the ring past the
  // slabs and the exchange, written after the main loop
  float* lnab = SPLITR ? reinterpret_cast<float*>(smem) + NW * 32 * slab_ld(TN) + XCH
                       : LdsFloats<EPI == EPI_LN ? 2 * BM : 0>::get();

  // the wave index is uniform: every LDS destination of the DMA loads is scalar arithmetic
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int g = lane >> 5, l32 = lane & 31;

  // Tile order, walked in groups of p.tgroup tile rows so that neighbouring tiles share A and W
  // panels. Blocks b, b+8, ... land on one XCD (round-robin dispatch): with p.tcontig each XCD
  // takes a contiguous run of tiles, else the round-robin deal (the launcher's choice).
  const int nblk = tiles_m * tiles_n;
  // split-K slices (EPI_PART): block b covers tile b % nblk over k-tiles [kt0, kt0 + nk)
  const int split = EPI == EPI_PART ? int(blockIdx.x) / nblk : 0;
  const int b0 = int(blockIdx.x) - split * nblk;
  const int bid = (EPI != EPI_PART && p.tcontig) ? xcd_contiguous(b0, nblk) : b0;
  const int tg = p.tgroup;
  const int per_group = tg * tiles_n;
  const int first_m = (bid / per_group) * tg;
  const int gsize = min(tiles_m - first_m, tg);
  const int tm = first_m + (bid % per_group) % gsize;
  const int tn = (bid % per_group) / gsize;
  const long m0 = long(tm) * BM, n0 = long(tn) * BN;

  // Each lane loads chunk c of tile row r = (i*4 + wave)*RPI + lane/CPR for instruction i; with
  // slot lane%CPR that chunk is slot ^ ((r >> SH) & (CPR-1)), the same for every i.
  const int lrow = lane / CPR;
  const int c = (lane % CPR) ^ (((wave * RPI + lrow) >> SH) & (CPR - 1));
  const int32x4_t rw = make_rsrc(p.W, uint32_t(long(p.N) * p.ldw * ES));
  uint32_t boff[BL];
#pragma unroll
  for (int i = 0; i < BL; ++i) {
    const long n = n0 + (i * NW + wave) * RPI + lrow;
    boff[i] = n < p.N ? uint32_t(n * p.ldw * ES + c * 16) : OOB;
  }
  int32x4_t ra;
  uint32_t aoff[AL];
  int aiy[AL], aix[AL];
  // Convolutions whose Cin is a multiple of BK: a k-tile lies inside one filter tap, so the tap
  // and its offset are uniform; each row keeps a bit mask of its in-bounds taps and its byte
  // offset at tap (0, 0) (modulo 2^32: the sum with a valid tap's offset is the real offset).
  constexpr bool conv_fast = AMODE == A_CONV_TAP;
  uint32_t tmsk[AL], rbase[AL];
  if (AMODE == A_ROWS) {
    ra = make_rsrc(p.A, uint32_t(long(p.M) * p.lda * ES));
#pragma unroll
    for (int i = 0; i < AL; ++i) {
      const long m = m0 + (i * NW + wave) * RPI + lrow;
      aoff[i] = m < p.M ? uint32_t(m * p.lda * ES + c * 16) : OOB;
    }
  } else {
    ra = make_rsrc(p.A, uint32_t(long(p.V) * p.Hi * p.Wi * p.Cin * ES));
    const int hw = p.Ho * p.Wo;
#pragma unroll
    for (int i = 0; i < AL; ++i) {
      const long m = m0 + (i * NW + wave) * RPI + lrow;
      if (m < p.M) {
        const int v = int(m / hw), rem = int(m - long(v) * hw);
        const int oy = rem / p.Wo, ox = rem - oy * p.Wo;
        aiy[i] = oy * p.stride - p.pad;
        aix[i] = ox * p.stride - p.pad;
        aoff[i] = uint32_t(long(v) * p.Hi * p.Wi * p.Cin * ES);
      } else {
        aiy[i] = -(1 << 20);
        aix[i] = 0;
        aoff[i] = 0;
      }
      tmsk[i] = 0;
      rbase[i] = 0;
      if (conv_fast && m < p.M) {
        rbase[i] = aoff[i] + uint32_t(((long(aiy[i]) * p.Wi + aix[i]) * p.Cin + c * KE) * ES);
        for (int ky = 0; ky < p.ks; ++ky)
          for (int kx = 0; kx < p.ks; ++kx) {
            const int iy = aiy[i] + ky, ix = aix[i] + kx;
            if (iy >= 0 && iy < p.Hi && ix >= 0 && ix < p.Wi) tmsk[i] |= 1u << (ky * p.ks + kx);
          }
      }
    }
  }

  const int nk_all = (p.K + BK - 1) / BK;
  const int kt0 = split * p.kper;
  const int nk = EPI == EPI_PART ? min(nk_all - kt0, p.kper) : nk_all;
  const int kend = min(p.K, (kt0 + nk) * BK);
  const int nk_full = (kend - kt0 * BK) / BK;  // k-tiles (from kt0) with every chunk inside [0, kend)
  // Load instruction l (l < AL: A rows, else W rows) of k-tile kt0 + kr into ring stage
  // `stage`. K-chunks at or past kend (tail and tiles beyond the slice) read as zeros. Row
  // operands put the k-tile offset in the scalar offset, so a load of a full k-tile (FULL:
  // kr < nk_full, known at compile time) costs no vector instruction; rows past the operand
  // have voffset OOB.
  auto issue_one = [&](int kr, int stage, int l, auto full) {
    constexpr bool FULL = decltype(full)::value;
    // A rows at sb + ..., W rows at sb + BM * RB + ... (split ring: A slot kr % AR, W slot `stage`)
    const uint32_t sb = SPLITR ? lds_addr(smem + (l < AL ? (kr % AR) * BM * RB : AR * BM * RB + stage * BN * RB - BM * RB))
                               : lds_addr(smem + stage * STAGE);
    const int kt = kt0 + kr;
    const int k = kt * BK + c * KE;
    const bool kin = FULL || k < kend;
    if (l < AL) {
      const int i = l;
      if (AMODE == A_ROWS) {
        load_to_lds(ra, kin ? aoff[i] : OOB, uint32_t(kt) * RB, sb + (i * NW + wave) * 1024);
      } else if constexpr (conv_fast) {
        // uniform: tap, ci0 and the tap's offset are scalars; a row whose tap is out of bounds
        // gets bit 31 set (every valid offset is below 2^31), a tile past kend voffset OOB
        const int kk = kt * BK;
        const int tap = kk / p.Cin, ci0 = kk - tap * p.Cin;
        const int ky = tap / p.ks, kx = tap - ky * p.ks;
        const uint32_t toff = __builtin_amdgcn_readfirstlane(int(((ky * p.Wi + kx) * p.Cin + ci0) * ES));
        const uint32_t bad = ((tmsk[i] >> (tap & 31)) & 1u) ^ 1u;
        uint32_t voff = (rbase[i] + toff) | (bad << 31);
        if (!FULL && kk >= kend) voff = OOB;
        load_to_lds(ra, voff, 0u, sb + (i * NW + wave) * 1024);
      } else {
        const int tap = k / p.Cin, ci = k - tap * p.Cin;
        const int ky = tap / p.ks, kx = tap - ky * p.ks;
        const int iy = aiy[i] + ky, ix = aix[i] + kx;
        const bool ok = kin && iy >= 0 && iy < p.Hi && ix >= 0 && ix < p.Wi;
        load_to_lds(ra, ok ? aoff[i] + uint32_t((iy * p.Wi + ix) * p.Cin + ci) * ES : OOB, 0u,
                    sb + (i * NW + wave) * 1024);
      }
    } else {
      const int i = l - AL;
      load_to_lds(rw, kin ? boff[i] : OOB, uint32_t(kt) * RB, sb + BM * RB + (i * NW + wave) * 1024);
    }
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // fragment rows are frow plus multiples of 32 (bf16: l32) or 16 (fp32: l%16)
  const int frow = L16 ? (lane & 15) : l32, fsub = L16 ? (lane >> 4) : g;
  const int sw = (frow >> SH) & (CPR - 1);
  const int arow0 = (wm * (BM / WM) + frow) * RB, brow0 = (BM + wn * (BN / WN) + frow) * RB;
  // byte offset of this lane's chunk in k-step s of a tile row
  auto step_off = [&](int st) { return (((L16 ? 4 : 2) * st + fsub) ^ sw) * 16; };
  // Prologue: AHEAD tiles in flight, tile 0 resident for every wave, its first fragments read.
  // Every k-tile slot is loaded, also past the last tile (as zeros), so that the number of
  // loads in flight, and with it each vmcnt wait, is the same for every tile.
  // With three or more stages (SPREAD) tile kt issues the loads of tile kt + STAGES - 1 during
  // its steps before the barrier step, into the stage that tile kt - 1 left: a DMA load holds
  // up the wave that issues it, so loads crowded into one step leave the matrix core idle (the
  // 6222x1024x4096 GEMM on 256x128 tiles: 61 -> 52 us). With two stages a stage frees only at
  // the barrier, and the loads of tile kt + 2 go into the barrier step.
  constexpr bool SPREAD = STAGES >= 3;
  constexpr int AHEAD = SPREAD ? STAGES - 1 : STAGES;  // tile kt loads tile kt + AHEAD
  // Folded LayerNorm: thread r < BM loads the partial statistics of tile row r ahead of the
  // operand tiles (up to 16 pairs) and reduces them once the first stage is resident.
  // The loads are unconditional (a clamped row and partial; the zeros are applied afterwards) so
  // that the compiler issues all of them back to back, not each behind its own wait.
  float2 lnv[EPI == EPI_LN ? 16 : 1];
  const long lnm = m0 + tid;
  if constexpr (EPI == EPI_LN) {
    const float* lrow = p.ln_in + (tid < BM && lnm < p.M ? lnm : 0) * p.ln_parts * 2;
#pragma unroll
    for (int j = 0; j < 16; ++j) lnv[j] = *reinterpret_cast<const float2*>(lrow + min(j, p.ln_parts - 1) * 2);
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if (j >= p.ln_parts) lnv[j] = make_float2(0.f, 0.f);
  }
  // Stage 0, then the row statistics (the compiler's wait for their loads also covers the DMA
  // loads issued before it, which tile 0 needs anyway), then the later stages.
#pragma unroll
  for (int l = 0; l < LPT; ++l) issue_one(0, 0, l, std::false_type{});
  float ln_rstd = 0.f, ln_shift = 0.f;
  if constexpr (EPI == EPI_LN) {
    if (tid < BM) {
      float s = 0.f, q = 0.f;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        s += lnv[j].x;
        q += lnv[j].y;
      }
      const float inv = 1.f / float(p.K), mean = s * inv;
      ln_rstd = rsqrtf(fmaxf(q * inv - mean * mean, 0.f) + p.ln_eps);
      ln_shift = -ln_rstd * mean;
      if constexpr (!SPLITR) {
        lnab[2 * tid] = ln_rstd;
        lnab[2 * tid + 1] = ln_shift;
      }
    }
  }
#pragma unroll
  for (int s = 1; s < AHEAD; ++s)
#pragma unroll
    for (int l = 0; l < LPT; ++l) issue_one(s, s, l, std::false_type{});
  wait_vmcnt<(AHEAD - 1) * LPT>();
  __syncthreads();
  // fp32 tiles share a CU two or four at a time: a block in its main loop issues ahead of a
  // block in its prologue or epilogue (C1 -0.3%; for the 16-bit tiles, mostly one a CU, the same
  // measured slower)
  if constexpr (sizeof(T) == 4) __builtin_amdgcn_s_setprio(1);
  // Fragments of the next k-step (of this tile, or step 0 of the next tile) are read while the
  // matrix cores work on the current one.
  uint4 fa[2][TM * FH], fb[2][TN * FH];
  // Fragment f of a k-step in the order the MFMAs (i outer, j inner) first use them: the A
  // fragments of tile row 0, then every W fragment, then the other A ones, so that the first
  // MFMAs of a step wait for few reads. Fragment rows are 32 / FH apart.
  // k-tile kt's A rows at abase(kt) + arow0.., its W rows at wbase(kt) + brow0.. (brow0 counts
  // the BM A rows of a whole stage)
  auto abase = [&](int kt) -> const char* { return smem + (SPLITR ? (kt % AR) * BM * RB : (kt % STAGES) * STAGE); };
  auto wbase = [&](int kt) -> const char* {
    return SPLITR ? smem + AR * BM * RB + (kt % STAGES) * BN * RB - BM * RB : smem + (kt % STAGES) * STAGE;
  };
  auto read_frag = [&](int kt, int off, int slot, int f) {
    constexpr int RS = 32 / FH * RB;
    const char* sa = abase(kt);
    const char* sw_ = wbase(kt);
    if (f < FH) fa[slot][f] = *reinterpret_cast<const uint4*>(sa + arow0 + f * RS + off);
    else if (f < FH + TN * FH) fb[slot][f - FH] = *reinterpret_cast<const uint4*>(sw_ + brow0 + (f - FH) * RS + off);
    else fa[slot][f - TN * FH] = *reinterpret_cast<const uint4*>(sa + arow0 + (f - TN * FH) * RS + off);
  };
  auto read_frags = [&](int kt, int s, int slot) {
    const int off = step_off(s);
#pragma unroll
    for (int f = 0; f < (TM + TN) * FH; ++f) read_frag(kt, off, slot, f);
  };
  // the products of tile pair (i, j) for the k-step whose fragments sit in `slot`
  auto mma = [&](int i, int j, int slot) {
    if constexpr (L16)
      Mfma<float>::mma2x2(acc[i][j], fa[slot][2 * i], fa[slot][2 * i + 1], fb[slot][2 * j], fb[slot][2 * j + 1]);
    else
      Mfma<T>::mma(acc[i][j], fa[slot][i], fb[slot][j]);
  };
  read_frags(0, 0, 0);
  // One k-tile; the last one is peeled (HAS_NEXT false) so that each step's reads and MFMAs
  // share a basic block and the LDS waits stay exact.
  constexpr int MM = TM * TN, NF = (TM + TN) * FH, CUR = (KS - 1) & 1;
  auto tile = [&](int kt, auto has_next, auto full) {
    constexpr bool HAS_NEXT = decltype(has_next)::value;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      // hard fence: the reads below belong to this step's region and nothing moves across
      __builtin_amdgcn_sched_barrier(0);
      if (RELU) {
#pragma unroll
        for (int i = 0; i < TM * FH; ++i) fa[s & 1][i] = Mfma<T>::relu(fa[s & 1][i]);
      }
      if ((SPREAD || (SPLITR && HAS_NEXT)) && s + 1 < KS) {
        // this step's share of the loads of tile kt + AHEAD (split ring: of the A rows of tile
        // kt + 2 only) and the reads of the next step's fragments, spread between the MFMAs
        constexpr int LS = SPLITR ? AL : LPT;
        const int L0 = s * LS / (KS - 1), L1 = (s + 1) * LS / (KS - 1);
        const int off = step_off(s + 1);
#pragma unroll
        for (int q = 0; q < MM; ++q) {
          mma(q / TN, q % TN, s & 1);
#pragma unroll
          for (int l = L0 + q * (L1 - L0) / MM; l < L0 + (q + 1) * (L1 - L0) / MM; ++l)
            issue_one(kt + AHEAD, (kt + AHEAD) % STAGES, l, full);
#pragma unroll
          for (int r = q * NF / MM; r < (q + 1) * NF / MM; ++r) read_frag(kt, off, (s + 1) & 1, r);
          __builtin_amdgcn_sched_barrier(0);
        }
      } else if (s + 1 < KS || !HAS_NEXT) {
        if (s + 1 < KS) read_frags(kt, s + 1, (s + 1) & 1);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) mma(i, j, s & 1);
        if (s + 1 < KS) {
          // interleave the LDS reads with this step's MFMAs
#pragma unroll
          for (int k = 0; k < NF; ++k) {
            __builtin_amdgcn_sched_group_barrier(0x008, MM * MPI / NF > 0 ? MM * MPI / NF : 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          }
        }
      } else {
        // Last step of a tile with a successor. Every wave holds its last fragments of tile kt
        // (the barrier waits for LDS reads), so the stage of tile kt is free once tile kt+1 is
        // resident (tiles kt+2 .. kt+STAGES-1 may still be in flight). With two stages the
        // loads of tile kt+2 and the reads of the next tile's first fragments are spread
        // between this step's MFMAs, in a fixed order; with more, only the reads.
        // Split ring: tile kt+1 is resident once at most the AL loads of A tile kt+2 are in
        // flight; then the W loads of tile kt+2 go out.
        wait_vmcnt<SPLITR ? AL : (STAGES - 2) * LPT>();
        __syncthreads();
        const int off0 = step_off(0);
        constexpr int LB = SPLITR ? AL : 0, LN_ = LPT - LB;
#pragma unroll
        for (int q = 0; q < MM; ++q) {
          mma(q / TN, q % TN, CUR);
          if constexpr (!SPREAD) {
#pragma unroll
            for (int l = LB + q * LN_ / MM; l < LB + (q + 1) * LN_ / MM; ++l) issue_one(kt + STAGES, kt % STAGES, l, full);
          }
#pragma unroll
          for (int r = q * NF / MM; r < (q + 1) * NF / MM; ++r) read_frag(kt + 1, off0, 0, r);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // tiles whose loads are of a full tile (kt + AHEAD), then the rest; the last is peeled
  int kt = 0;
  for (; kt + 1 < nk && kt + AHEAD < nk_full; ++kt) tile(kt, std::true_type{}, std::true_type{});
  for (; kt + 1 < nk; ++kt) tile(kt, std::true_type{}, std::false_type{});
  tile(nk - 1, std::false_type{}, std::false_type{});
  wait_vmcnt<0>();  // the zero-fill loads past the last tile must land before the ring is reused
  __syncthreads();  // every wave is past its last read of the ring before slabs reuse it
  if constexpr (SPLITR && EPI == EPI_LN) {
    if (tid < BM) {
      lnab[2 * tid] = ln_rstd;
      lnab[2 * tid + 1] = ln_shift;
    }
    __syncthreads();
  }
  if constexpr (sizeof(T) == 4) __builtin_amdgcn_s_setprio(0);
  if constexpr (EPI == EPI_HEAD) {
    static_assert(NW * 32 * slab_ld(TN) * 4 + BM * WN * 6 * 4 <= RING, "head epilogue LDS");
    head_epilogue<T, BM, BN, WM, WN, TM, TN, L16>(p, acc, m0, wm, wn, reinterpret_cast<float*>(smem), wave, lane, tid);
  } else {
    float* slab = reinterpret_cast<float*>(smem) + wave * 32 * slab_ld(TN);
    constexpr int LNLD = BN / 32;  // 32-column sums per tile row (EPI_RESLN)
    float* lnp = reinterpret_cast<float*>(smem) + NW * 32 * slab_ld(TN);
    epilogue<T, TM, TN, EPI, L16>(p, acc, m0 + wm * (BM / WM), n0 + wn * (BN / WN), slab, lane, p.epi_vec,
                             EPI == EPI_PART ? p.part + long(split) * p.M * p.ldp : nullptr,
                             EPI == EPI_LN ? lnab + wm * (BM / WM) * 2 : nullptr,
                             lnp + (wm * (BM / WM) * LNLD + wn * (BN / WN) / 32) * 2, LNLD,
                             lnp + (wn / 2) * BM * 4, wm * (BM / WM));
    if constexpr (EPI == EPI_RESLN) {
      // every wave's 32-column sums are in LDS: one (sum, sum of squares) per row and group
      __syncthreads();
      const int gw = p.ln_group / 32, ng = BN / p.ln_group, parts = p.N / p.ln_group;
      for (int idx = tid; idx < BM * ng; idx += NW * 64) {
        const int r = idx / ng, gg = idx - r * ng;
        const long m = m0 + r, nc = n0 + gg * p.ln_group;
        if (m < p.M && nc < p.N) {
          const float* a = lnp + (r * LNLD + gg * gw) * 2;
          float s = 0.f, q = 0.f;
          for (int c = 0; c < gw; ++c) {
            s += a[2 * c];
            q += a[2 * c + 1];
          }
          *reinterpret_cast<float2*>(p.ln_out + (m * parts + nc / p.ln_group) * 2) = make_float2(s, q);
        }
      }
    }
  }
}

// Split-K reduction: out = epilogue(sum over slices of the fp32 partials), 8 columns a thread.
template <typename T>
__global__ void __launch_bounds__(256) splitk_reduce_kernel(const GemmArgs p, int S, int stats) {
  const long runs = (p.N + 7) / 8;
  const long id = long(blockIdx.x) * 256 + threadIdx.x;
  if (id >= long(p.M) * runs) return;
  const long m = id / runs, n = (id - m * runs) * 8;
  const long stride = long(p.M) * p.ldp;
  const float* src = p.part + m * p.ldp + n;
  float v[8];
  read8(src, v);
  for (int s = 1; s < S; ++s) {
    float w[8];
    read8(src + s * stride, w);
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] += w[k];
  }
  epi8<T>(p, v, m, n, p.epi_vec && n + 8 <= p.N);
  if (stats) {
    // A producer's row statistics (and copy) of the stored rows: a group of ln_group columns is
    // ln_group / 8 consecutive lanes (N a multiple of the group, so groups are lane-aligned and
    // whole), summed by DPP; the group's first lane writes the (sum, sum of squares) pair.
    float sm = 0.f, sq = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      sm += v[k];
      sq = fmaf(v[k], v[k], sq);
    }
    if (p.ln_group == 64) {
      sm = group_sum<8>(sm);
      sq = group_sum<8>(sq);
    } else {
      sm = group_sum<16>(sm);
      sq = group_sum<16>(sq);
    }
    if ((n % p.ln_group) == 0)
      *reinterpret_cast<float2*>(p.ln_out + (m * (p.N / p.ln_group) + n / p.ln_group) * 2) = make_float2(sm, sq);
    if (p.ln_copy) store8_to<T>(p.ln_copy, false, v, m * p.ldc + n);
  }
}

constexpr int GEMM_CUS = 256;  // MI355X compute units: one "round" of resident blocks per CU slot

// XCD-aware tile map of a row GEMM. The 8 XCDs have an L2 each, so a launch fetches into each
// L2 the A panels of the tile rows and the W panels of the tile columns that the XCD's blocks
// touch (each panel BM or BN rows by K). Among tile-group heights 8, 1 and ceil(tm / r) for
// r = 2, 4, 8, each with contiguous runs and with the round-robin deal, take the map whose
// blocks touch the fewest panel rows (BM per tile row plus BN per tile column, summed over the
// XCDs); ties keep 8-row groups and the deal the tile count gave before. Encoder qkv at C4
// (20 x 12 tiles of 320x256): 67.9 -> 51.4 MB of panels (groups of 5 rows: each XCD a 5 x 6
// block); fc2 (25 x 8 tiles of 256x128, K = 4096): 197 -> 134 MB. Cached per shape. Only for
// launches of at most two rounds, whose blocks run nearly all at once: over more rounds the
// order in time matters more than the union of panels (8192^3, four rounds: contiguous runs
// 1.30 PFLOP/s, the round-robin deal 1.01), so those keep the default.
struct XcdTileMap { int tm, tn, bm, bn, group, contig; };
static void xcd_tile_map(GemmArgs& b, int tm, int tn, int bm, int bn) {
  const int nblk = tm * tn;
  if (nblk > 2 * GEMM_CUS) return;
  static thread_local std::vector<XcdTileMap> cache;
  for (const XcdTileMap& c : cache)
    if (c.tm == tm && c.tn == tn && c.bm == bm && c.bn == bn) {
      b.tgroup = c.group;
      b.tcontig = c.contig;
      return;
    }
  std::vector<char> rows(size_t(8) * tm), cols(size_t(8) * tn);
  auto cost = [&](int g, bool contig) {
    std::fill(rows.begin(), rows.end(), 0);
    std::fill(cols.begin(), cols.end(), 0);
    long c = 0;
    for (int blk = 0; blk < nblk; ++blk) {
      const int x = blk & 7, bid = contig ? xcd_contiguous(blk, nblk) : blk;
      const int per_group = g * tn, first = (bid / per_group) * g, gs = std::min(tm - first, g);
      const int r = first + (bid % per_group) % gs, q = (bid % per_group) / gs;
      if (!rows[size_t(x) * tm + r]) { rows[size_t(x) * tm + r] = 1; c += bm; }
      if (!cols[size_t(x) * tn + q]) { cols[size_t(x) * tn + q] = 1; c += bn; }
    }
    return c;
  };
  int best_g = b.tgroup, best_contig = b.tcontig;
  long best = cost(best_g, best_contig);
  const int gs[] = {8, 1, cdiv(tm, 2), cdiv(tm, 4), cdiv(tm, 8)};
  for (int g : gs)
    for (int contig = 1; contig >= 0; --contig) {
      if (g < 1) continue;
      const long c = cost(g, contig);
      if (c < best) { best = c; best_g = g; best_contig = contig; }
    }
  b.tgroup = best_g;
  b.tcontig = best_contig;
  cache.push_back({tm, tn, bm, bn, best_g, best_contig});
}

// TAP_ONLY: an instantiation that serves per-tap convolutions only (the 32-element k-tiles for
// maps whose Cin is a multiple of 32 but not of 64).
// Returns whether the launch wrote the row statistics (and copy) a producer (ln_out) asks for.
template <typename T, int BM, int BN, int WM, int WN, int STAGES, int BK = 128 / sizeof(T), int MINB = 1,
          bool TAP_ONLY = false, int AR = STAGES>
static bool launch_mfma(const Exec& ex, const GemmArgs& a, int S) {
  static_assert(MINB == 1 || MINB * STAGES * (BM + BN) * BK * sizeof(T) <= 160 * 1024, "LDS of MINB blocks per CU");
  const int tm = cdiv(a.M, BM), tn = cdiv(a.N, BN);
  int epi = S > 1 ? EPI_PART : epi_kind(a);
  if (epi == EPI_RESLN && (a.amode != A_ROWS || TAP_ONLY || BN % a.ln_group != 0)) epi = EPI_RES;  // statistics afterwards
  SPLAT_CHECK(!a.ln_in || (epi == EPI_LN && a.amode == A_ROWS && !TAP_ONLY), BAD_ARGUMENT,
              "gemm: a folded LayerNorm needs plain rows, a vectorisable epilogue and no split-K");
  GemmArgs b = a;
  b.tgroup = 8;
  // Convolutions: each XCD takes a contiguous run of tiles, i.e. a band of output rows, so the
  // halo rows two neighbouring tiles share are fetched into one L2 (xcd_contiguous spreads a tile
  // count that is not a multiple of 8 over the XCDs in runs that differ by at most one tile).
  b.tcontig = a.amode != A_ROWS || (tm * tn) % 8 == 0;
  if (a.amode == A_ROWS && S == 1) xcd_tile_map(b, tm, tn, BM, BN);
  if (S > 1) {
    b.part = static_cast<float*>(ex.ws->ptr);
    b.ldp = (a.N + 7) / 8 * 8;
    b.kper = cdiv(cdiv(a.K, BK), S);
  }
  dim3 grid(tm * tn * S);
#define SPLAT_GO(AM, RL, EP) \
  hipLaunchKernelGGL((gemm_mfma_kernel<T, BM, BN, WM, WN, STAGES, BK, AM, RL, EP, MINB, AR>), grid, dim3(WM * WN * 64), 0, ex.stream, \
                     b, tm, tn)
  // Convolutions take the per-tap path (A_CONV_TAP) when Cin is a multiple of the k-tile, else
  // the per-lane im2col arithmetic (A_CONV, without ReLU-on-load: no such caller).
  const bool tap = a.amode == A_CONV && a.Cin % BK == 0 && a.ks * a.ks <= 32;
  SPLAT_CHECK(a.amode == A_ROWS || tap || !a.relu_in, BAD_ARGUMENT,
              "gemm: ReLU-on-load needs a convolution whose Cin is a multiple of the k-tile");
  if (TAP_ONLY) SPLAT_CHECK(tap && epi != EPI_HEAD, BAD_ARGUMENT, "gemm: 32-element k-tiles serve per-tap convs only");
  if (epi == EPI_HEAD) {  // the fused MapAnything head: one tile spans the 128 channels
    SPLAT_CHECK(tap && !a.relu_in && a.N == BN && a.act == ACT_RELU && S == 1, BAD_ARGUMENT, "gemm: fused head");
    if constexpr (BN == 128 && sizeof(T) == 2 && !TAP_ONLY) SPLAT_GO(A_CONV_TAP, false, EPI_HEAD);
    else SPLAT_CHECK(false, BAD_ARGUMENT, "gemm: fused head needs a bf16 128-column tile");
  } else if (a.amode == A_ROWS) {
    if constexpr (!TAP_ONLY) {
      if (epi == EPI_PART) SPLAT_GO(A_ROWS, false, EPI_PART);
      else if (epi == EPI_BIAS) SPLAT_GO(A_ROWS, false, EPI_BIAS);
      else if (epi == EPI_RES) SPLAT_GO(A_ROWS, false, EPI_RES);
      else if (epi == EPI_LN) SPLAT_GO(A_ROWS, false, EPI_LN);
      else if (epi == EPI_RESLN) SPLAT_GO(A_ROWS, false, EPI_RESLN);
      else SPLAT_GO(A_ROWS, false, EPI_FULL);
    }
  } else if (tap) {
    if (epi == EPI_PART) {
      if (a.relu_in) SPLAT_GO(A_CONV_TAP, true, EPI_PART);
      else SPLAT_GO(A_CONV_TAP, false, EPI_PART);
    } else if (epi == EPI_BIAS) {
      if (a.relu_in) SPLAT_GO(A_CONV_TAP, true, EPI_BIAS);
      else SPLAT_GO(A_CONV_TAP, false, EPI_BIAS);
    } else if (epi == EPI_RES && !a.relu_in) {  // the residual units' second conv
      SPLAT_GO(A_CONV_TAP, false, EPI_RES);
    } else {
      if (a.relu_in) SPLAT_GO(A_CONV_TAP, true, EPI_FULL);
      else SPLAT_GO(A_CONV_TAP, false, EPI_FULL);
    }
  } else {
    if constexpr (!TAP_ONLY) {
      if (epi == EPI_PART) SPLAT_GO(A_CONV, false, EPI_PART);
      else if (epi == EPI_BIAS) SPLAT_GO(A_CONV, false, EPI_BIAS);
      else SPLAT_GO(A_CONV, false, EPI_FULL);
    }
  }
#undef SPLAT_GO
  SPLAT_HIP(hipGetLastError());
  // the reduce of a split producer emits its row statistics too (whole 8-column runs, plain rows)
  const bool rstats = S > 1 && a.ln_out && a.epi_vec && !a.rm_P && a.store == STORE_ROWS &&
                      (a.ln_group == 64 || a.ln_group == 128) && a.N % a.ln_group == 0;
  if (S > 1) {
    const long work = long(a.M) * ((a.N + 7) / 8);
    hipLaunchKernelGGL(splitk_reduce_kernel<T>, dim3(unsigned((work + 255) / 256)), dim3(256), 0, ex.stream, b, S,
                       int(rstats));
    SPLAT_HIP(hipGetLastError());
  }
  return epi == EPI_RESLN || rstats;
}

// Tile configurations of the bf16 path: block tile, and how many blocks share a CU.
enum BfCfg { CFG_128x32, CFG_128x64, CFG_256x256, CFG_256x128, CFG_320x256, CFG_320x128, CFG_192x128, CFG_128x128,
             CFG_F128x128, CFG_F64x64, CFG_192x128D };
struct BfShape { int bm, bn, per_cu; };
static BfShape bf_shape(BfCfg c) {
  switch (c) {
    case CFG_128x32: return {128, 32, 3};
    case CFG_128x64: return {128, 64, 3};
    case CFG_256x256: return {256, 256, 1};
    case CFG_256x128: return {256, 128, 1};
    case CFG_320x256: return {320, 256, 1};
    case CFG_320x128: return {320, 128, 1};
    case CFG_192x128: return {192, 128, 1};
    case CFG_F128x128: return {128, 128, 2};
    case CFG_F64x64: return {64, 64, 4};
    case CFG_192x128D: return {192, 128, 2};
    default: return {128, 128, 1};
  }
}

// Tile choice: the fewest "rounds" of 256 CUs weighted by a per-tile cost relative to the
// 256x256 tile (smaller tiles re-read more operand bytes through LDS per flop). The 256-row
// tiles run 8 waves, two per SIMD: while one wave waits on its LDS reads the other issues
// MFMAs, which the one-wave-per-SIMD form cannot hide (network shapes of the MapAnything C4
// encoder, bias epilogue: 391 -> 331 us summed over one block's eight GEMMs). The other
// shapes exist for the round count at M = 5838-6223 rows, where 256-row tiles leave a last
// round mostly empty: 320x256 (8 waves of 160x64, 2 stages) puts 6222x3072 in one round of 240
// tiles (QKV 6222x3072x1024: 59.5 us as 600 tiles of 256x128, 48.5 as 480 of 320x128, 42.3);
// 192x128 (8 waves of 96x32, 3 stages) puts N = 768 in one round of 198 smaller tiles
// (6223x768x3072 42.4 -> 38.4 us).
static BfCfg pick_bf16(const GemmArgs& a) {
  // Narrow outputs (the DA3 head's 32/64-channel convs): 128-row tiles and two stages keep the
  // LDS per block at 40-48 KB, so 3-4 blocks share a CU and hide each other's load latency
  // (C2 convs 475 -> 266 us against 256-row tiles with 3-4 stages).
  if (a.N <= 32 && !a.qk_dim) return CFG_128x32;
  if (a.N <= 64 && !a.qk_dim) return CFG_128x64;
  // 128-channel convolutions over many tiles (the DPT heads' output convs at full and half
  // resolution): 192x128 tiles with two stages, 80 KB of LDS, so that two blocks share a CU and
  // one block's prologue and epilogue overlap the other's main loop. Measured from 1.5 rounds of
  // such blocks up (3x3, 128 -> 128: M = 173k 75 -> 64 us, 1.2M 475-497 -> 443 us; 256 -> 128 at
  // M = 398k 321 -> 284 us); below ~100k pixels the smaller tiles lose (25k: 18.4 -> 19.4 us).
  if (a.amode == A_CONV && a.N == 128 && cdiv(a.M, 192) >= 3 * GEMM_CUS) return CFG_192x128D;
  const BfCfg cands[] = {CFG_256x256, CFG_256x128, CFG_320x256, CFG_320x128, CFG_192x128, CFG_128x128};
  const double eff[] = {1.0, 0.80, 1.0, 0.80, 0.75, 0.65};
  // On equal cost the fewer, larger rounds win (MapAnything C5's 24888x3072x1024 qkv: five
  // rounds of 256x256 or four of 320x256, 191 -> 172 us).
  double best = 1e30;
  long best_rounds = 0;
  BfCfg pick = a.hw3 ? CFG_320x128 : CFG_256x256;
  for (int i = 0; i < 6; ++i) {
    const BfShape sh = bf_shape(cands[i]);
    if (a.hw3 && sh.bn != 128) continue;  // the fused head needs the 128 channels in one tile
    const long tiles = long(cdiv(a.M, sh.bm)) * cdiv(a.N, sh.bn);
    const long rounds = (tiles + GEMM_CUS - 1) / GEMM_CUS;
    const double cost = double(rounds) * sh.bm * sh.bn / eff[i];
    if (cost < best * 0.999 || (cost <= best * 1.001 && rounds < best_rounds)) {
      best = cost;
      best_rounds = rounds;
      pick = cands[i];
    }
  }
  return pick;
}

// Split-K: a launch whose tiles fill less than half of one round of block slots and whose K
// spans at least 16 k-tiles is cut into S >= 2 slices of at least 8 k-tiles, S * tiles within
// one round. The slices write fp32 partials; a second kernel sums them and applies the
// epilogue (the DPT head's coarse-level convs: M = 1596, K = 6912, 14 tiles of 256x128).
static int split_factor(const GemmArgs& a, BfCfg c) {
  if (a.hw3 || a.ln_in) return 1;  // the fused head needs whole tiles, a folded LayerNorm whole rows of K
  const BfShape sh = bf_shape(c);
  const long tiles = long(cdiv(a.M, sh.bm)) * cdiv(a.N, sh.bn);
  const long slots = long(GEMM_CUS) * sh.per_cu;
  const int nk = cdiv(a.K, a.dt == F32 ? 32 : 64);
  if (2 * tiles > slots || nk < 16) return 1;
  const int S = int(std::min<long>(nk / 8, slots / tiles));
  if (S < 2) return 1;
  return cdiv(nk, cdiv(nk, S));  // every slice non-empty
}
static size_t split_bytes(const GemmArgs& a, int S) {
  return S > 1 ? size_t(S) * a.M * ((a.N + 7) / 8 * 8) * sizeof(float) : 0;
}

// fp32 (every GEMM of the fp32 mode): the matrix cores run fp32 at 1/16 of the bf16 rate, so
// operand traffic is minor and the tile choice only has to fill the CUs: a round of resident
// tiles runs per_cu tiles per CU side by side, so its cost is per_cu x the tile's area.
static BfCfg pick_f32(const GemmArgs& a) {
  if (a.N <= 32 && !a.qk_dim) return CFG_128x32;
  if (a.N <= 64 && !a.qk_dim) return CFG_F64x64;
  const BfCfg cands[] = {CFG_256x256, CFG_256x128, CFG_F128x128, CFG_F64x64};
  double best = 1e30;
  BfCfg pick = CFG_256x256;
  for (BfCfg c : cands) {
    const BfShape sh = bf_shape(c);
    const long tiles = long(cdiv(a.M, sh.bm)) * cdiv(a.N, sh.bn);
    const long slots = long(GEMM_CUS) * sh.per_cu;
    const double cost = double((tiles + slots - 1) / slots) * sh.per_cu * sh.bm * sh.bn;
    if (cost < best * 0.999) { best = cost; pick = c; }
  }
  return pick;
}

static bool launch_f32_auto(const Exec& ex, const GemmArgs& a) {
  const BfCfg c = pick_f32(a);
  int S = split_factor(a, c);
  if (S > 1 && !(ex.ws && ex.ws->ptr && ex.ws->cap >= split_bytes(a, S))) S = 1;
  switch (c) {
    case CFG_128x32: return launch_mfma<float, 128, 32, 4, 1, 2>(ex, a, S);
    case CFG_256x256: return launch_mfma<float, 256, 256, 2, 4, 2>(ex, a, S);
    case CFG_256x128: return launch_mfma<float, 256, 128, 4, 2, 3>(ex, a, S);
    case CFG_F128x128: return launch_mfma<float, 128, 128, 2, 2, 2>(ex, a, S);
    default: return launch_mfma<float, 64, 64, 2, 2, 2>(ex, a, S);
  }
}

// ---------------------------------------------------------------------------------------------
// 3x3 stride-1 convolutions with Cin and Cout in {32, 64}, 16-bit types: the DPT heads of the
// small models (the fusion units, output and ray convolutions of DA3-Small, up to full image
// resolution). On the per-tap tiles these read every input pixel nine times through the load
// path for only 32-64 output channels. Here a persistent block keeps the whole filter
// [Cout][9 Cin] in LDS and walks output tiles of 8 rows x 32 columns of one view: each tile's
// input halo (10 x 34 pixels, zeros outside the view) streams into one of NBUF LDS buffers
// ahead of its use, and the nine taps take their A fragments from the halo at shifted pixels.
// Eight compute waves, one tile row each, Cout / 32 accumulators of 32 pixels x 32 channels,
// and a ninth wave that only issues the direct-to-LDS loads (filter, halos) and waits for them,
// so that the compute waves never wait on the memory counter: their epilogue loads and stores
// stay in flight across tiles. Two block barriers a tile: A (the tile's halo is resident) and C
// (every compute wave is past its reads of it). The loader issues tile it + NBUF - 1's halo
// after barrier A of tile it, into the buffer that tile it - 1 left (its epilogue slabs, staged
// in its own halo buffer, were done before barrier A).
// LDS: filter rows of 9 Cin elements padded to an odd number of 16-byte chunks, so that the 16
// rows of a fragment-read phase land on 16 distinct 4-bank groups; halo pixel q keeps chunk c in
// slot c ^ ((q >> SHP) & (CPP - 1)), so that 16 consecutive pixels do.
template <typename T, int CIN, int COUT, bool RELU>
__global__ void __launch_bounds__(576, 1) conv3x3_halo_kernel(const GemmArgs p, int tiles_x, int tiles_y) {
  constexpr int TH = 8, TW = 32, HC = TW + 2, HR = TH + 2;
  constexpr int CPP = CIN * 2 / 16;  // 16-byte chunks a pixel: 8 or 4
  constexpr int SHP = CPP == 8 ? 1 : 2;
  constexpr int HCH = HR * HC * CPP;  // chunks of a halo
  constexpr int NDMA = (HCH + 63) / 64;  // DMA instructions a halo, 1 KiB each
  constexpr int HBUF = NDMA * 1024;
  constexpr int WCH = 9 * CIN * 2 / 16, WCHP = WCH | 1;  // chunks of a filter row, and its LDS stride
  constexpr int WLD = WCHP * 16;
  constexpr int WDMA = (COUT * WCHP + 63) / 64;
  constexpr int HALO0 = WDMA * 1024;
  constexpr int NBUF = CIN == 64 ? 2 : 3;
  constexpr int SLD = slab_ld(1);
  constexpr int STG = 8 * 32 * SLD * 4;  // the eight compute waves' epilogue slabs
  constexpr bool STG_IN_HALO = HBUF >= STG;
  constexpr int LDS = HALO0 + NBUF * HBUF + (STG_IN_HALO ? 0 : STG);
  static_assert(LDS <= 160 * 1024, "LDS");
  static_assert(NDMA <= 63, "vmcnt range");
  __shared__ __attribute__((aligned(1024))) char smem[LDS];

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int per_view = tiles_x * tiles_y, tiles = p.V * per_view;
  const int G = gridDim.x, t0 = blockIdx.x;
  if (t0 >= tiles) return;  // the launcher sizes the grid to at most the tile count
  const int ntile = (tiles - t0 + G - 1) / G;  // this block's tiles: t0, t0 + G, ...

  const int32x4_t ra = make_rsrc(p.A, uint32_t(long(p.V) * p.Hi * p.Wi * CIN * 2));
  // Halo of the block's tile it: its origin (view v, input pixel (y0, x0)) and LDS buffer.
  auto tile_origin = [&](int it, int& y0, int& x0, int& ob) {
    const int u = t0 + it * G;
    const int v = u / per_view, r = u - v * per_view, ty = r / tiles_x, tx = r - ty * tiles_x;
    y0 = ty * TH - 1;
    x0 = tx * TW - 1;
    ob = ((v * p.Hi + y0) * p.Wi + x0) * (CIN * 2);  // byte offset of the origin (negative at a border)
  };
  // DMA instruction ins of a halo: lane chunk q = 64 ins + lane, halo pixel px = q / CPP at
  // (hr, hc), its slot q % CPP holding chunk slot ^ ((px >> SHP) & (CPP - 1)) of the pixel
  auto halo_lane = [&](int ins, int& hr, int& hc, int& rel) {
    const int q = ins * 64 + lane, px = q / CPP, sl = q - px * CPP;
    hr = q < HCH ? px / HC : HR;  // HR: a chunk past the halo, read as zeros
    hc = px - (px / HC) * HC;
    rel = ((px / HC) * p.Wi + hc) * (CIN * 2) + (sl ^ ((px >> SHP) & (CPP - 1))) * 16;
  };
  {
    // prologue, every wave: its share of the filter (LDS chunk q = row n, chunk c; the padding
    // chunk reads as zeros) and of tile 0's halo
    const int32x4_t rw = make_rsrc(p.W, uint32_t(long(p.N) * p.ldw * 2));
    for (int ins = wave; ins < WDMA; ins += 9) {
      const int q = ins * 64 + lane, n = q / WCHP, c = q - n * WCHP;
      const uint32_t off = (n < COUT && c < WCH) ? uint32_t(long(n) * p.ldw * 2 + c * 16) : OOB;
      load_to_lds(rw, off, 0u, lds_addr(smem) + ins * 1024);
    }
    int y0, x0, ob;
    tile_origin(0, y0, x0, ob);
    for (int ins = wave; ins < NDMA; ins += 9) {
      int hr, hc, rel;
      halo_lane(ins, hr, hc, rel);
      const bool ok = hr < HR && unsigned(y0 + hr) < unsigned(p.Hi) && unsigned(x0 + hc) < unsigned(p.Wi);
      load_to_lds(ra, ok ? uint32_t(ob + rel) : OOB, 0u, lds_addr(smem + HALO0) + ins * 1024);
    }
    wait_vmcnt<0>();
    __syncthreads();  // the filter and tile 0's halo are resident
  }

  if (wave == 8) {
    // loader wave: each DMA lane's halo pixel and relative offset, once
    int lhr[NDMA], lhc[NDMA], lrel[NDMA];
#pragma unroll
    for (int ins = 0; ins < NDMA; ++ins) halo_lane(ins, lhr[ins], lhc[ins], lrel[ins]);
    auto issue_halo = [&](int it) {
      int y0, x0, ob;
      tile_origin(it, y0, x0, ob);
      const uint32_t base = lds_addr(smem + HALO0 + (it % NBUF) * HBUF);
      if (y0 >= 0 && y0 + HR <= p.Hi && x0 >= 0 && x0 + HC <= p.Wi) {  // interior tile: every pixel inside
#pragma unroll
        for (int ins = 0; ins < NDMA; ++ins)
          load_to_lds(ra, lhr[ins] < HR ? uint32_t(ob + lrel[ins]) : OOB, 0u, base + ins * 1024);
      } else {
#pragma unroll
        for (int ins = 0; ins < NDMA; ++ins) {
          const bool ok = lhr[ins] < HR && unsigned(y0 + lhr[ins]) < unsigned(p.Hi) &&
                          unsigned(x0 + lhc[ins]) < unsigned(p.Wi);
          load_to_lds(ra, ok ? uint32_t(ob + lrel[ins]) : OOB, 0u, base + ins * 1024);
        }
      }
    };
    for (int it = 1; it < NBUF - 1 && it < ntile; ++it) issue_halo(it);
    for (int it = 0; it < ntile; ++it) {
      // tile it's halo has landed once only the halos issued after it may be in flight (tile 0's
      // landed in the prologue)
      const int later = min(ntile - 1 - it, NBUF - 2);
      if (later >= 1) wait_vmcnt<NDMA>();
      else wait_vmcnt<0>();
      __syncthreads();  // A
      if (it + NBUF - 1 < ntile) issue_halo(it + NBUF - 1);
      __syncthreads();  // C
    }
    return;
  }

  // compute waves
  const int g = lane >> 5, l32 = lane & 31;
  // per-lane bias: channels j * 32 + (lane & 3) * 8 + 0..7
  float bs[COUT / 32][8];
#pragma unroll
  for (int j = 0; j < COUT / 32; ++j) {
    const int n = j * 32 + (lane & 3) * 8;
#pragma unroll
    for (int k = 0; k < 8; ++k) bs[j][k] = p.bias ? p.bias[n + k] : 0.f;
  }
  const bool rf = p.res_f32 != 0, rf2 = p.res2_f32 != 0;
  for (int it = 0; it < ntile; ++it) {
    const int t = t0 + it * G;
    const int cur = it % NBUF;
    __syncthreads();  // A: this tile's halo is resident
    f32x16 acc[COUT / 32];
#pragma unroll
    for (int j = 0; j < COUT / 32; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[j][r] = 0.f;
    const char* hb = smem + HALO0 + cur * HBUF;
    // k-step s = (tap, 16-channel group kk); its fragments are read two steps ahead into one of
    // three register slots, so that the LDS latency hides behind two steps of MFMAs
    constexpr int KK = CIN / 16, NSTEP = 9 * KK, NJ = COUT / 32, PF = 2;
    uint4 fa[PF + 1], fb[PF + 1][NJ];
    auto read_step = [&](int st, int slot) {
      const int tap = st / KK, kk = st - tap * KK;
      const int px = (wave + tap / 3) * HC + l32 + tap % 3;  // halo pixel of this lane's A row
      const int c = 2 * kk + g;
      fa[slot] = *reinterpret_cast<const uint4*>(hb + (px * CPP + (c ^ ((px >> SHP) & (CPP - 1)))) * 16);
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        fb[slot][j] = *reinterpret_cast<const uint4*>(smem + (j * 32 + l32) * WLD + (tap * (CIN / 8) + c) * 16);
    };
#pragma unroll
    for (int st = 0; st < PF; ++st) read_step(st, st);
#pragma unroll
    for (int st = 0; st < NSTEP; ++st) {
      __builtin_amdgcn_sched_barrier(0);
      if (st + PF < NSTEP) {
        read_step(st + PF, (st + PF) % (PF + 1));
        __builtin_amdgcn_sched_group_barrier(0x100, 1 + NJ, 0);  // the reads first
      }
      uint4 a = fa[st % (PF + 1)];
      if constexpr (RELU) a = Mfma<T>::relu(a);
#pragma unroll
      for (int j = 0; j < NJ; ++j) Mfma<T>::mma(acc[j], a, fb[st % (PF + 1)][j]);
      __builtin_amdgcn_sched_barrier(0);
    }
    __syncthreads();  // C: every compute wave is past its reads of this halo
    float* slab = reinterpret_cast<float*>(smem + HALO0 + (STG_IN_HALO ? cur * HBUF : NBUF * HBUF)) + wave * 32 * SLD;
    const int v = t / per_view, r = t - v * per_view, ty = r / tiles_x, tx = r - ty * tiles_x;
    const int oy = ty * TH + wave;
    // the epilogue of GemmArgs (epi8's order; no LayerScale on this path): bias, act, table,
    // residuals, act_post
#pragma unroll
    for (int j = 0; j < COUT / 32; ++j) {
      // accumulator layout: lane l, register r -> pixel 8 (r / 4) + 4 (l / 32) + r % 4, channel l % 32
#pragma unroll
      for (int r2 = 0; r2 < 16; ++r2) slab[(8 * (r2 >> 2) + 4 * g + (r2 & 3)) * SLD + l32] = acc[j][r2];
      slab_done();
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int pix = (lane + 64 * h) >> 2, n = j * 32 + (lane & 3) * 8;
        const int ox = tx * TW + pix;
        if (oy < p.Ho && ox < p.Wo) {
          const long m = (long(v) * p.Ho + oy) * p.Wo + ox;
          float x[8], tt[8];
          read8(slab + pix * SLD + (lane & 3) * 8, x);
#pragma unroll
          for (int k = 0; k < 8; ++k) x[k] += bs[j][k];
          if (p.act == ACT_RELU) for (int k = 0; k < 8; ++k) x[k] = fmaxf(x[k], 0.f);
          else if (p.act == ACT_GELU) for (int k = 0; k < 8; ++k) x[k] = gelu_erf(x[k]);
          if (p.addtab) { load8<T>(p.addtab, (m % p.addtab_period) * p.N + n, true, tt); for (int k = 0; k < 8; ++k) x[k] += tt[k]; }
          if (p.res) { load8<T>(p.res, m * p.ldres + n, rf, tt); for (int k = 0; k < 8; ++k) x[k] += tt[k]; }
          if (p.res2) { load8<T>(p.res2, m * p.ldres2 + n, rf2, tt); for (int k = 0; k < 8; ++k) x[k] += tt[k]; }
          if (p.act_post == ACT_GELU) for (int k = 0; k < 8; ++k) x[k] = gelu_erf(x[k]);
          else if (p.act_post == ACT_RELU) for (int k = 0; k < 8; ++k) x[k] = fmaxf(x[k], 0.f);
          store8<T>(p, x, m * p.ldc + n);
        }
      }
      slab_done();
    }
  }
}

// Which convolutions take conv3x3_halo_kernel: 3x3, stride 1, padding 1, Cin and Cout 32 or 64,
// plain row stores without LayerScale, 16-byte aligned epilogue operands, and rows of at least
// 64 pixels (narrower maps waste most of a 32-column tile).
static bool conv_halo_ok(const GemmArgs& a) {
  return a.amode == A_CONV && a.ks == 3 && a.stride == 1 && a.pad == 1 && a.Ho == a.Hi && a.Wo == a.Wi &&
         (a.Cin == 32 || a.Cin == 64) && (a.N == 32 || a.N == 64) && a.store == STORE_ROWS && !a.rm_P && !a.hw3 &&
         !a.ln_in && !a.ln_out && !a.qk_dim && !a.glu && !a.q_cols && !a.gamma && a.epi_vec && a.Wo >= 64 &&
         double(a.V) * a.Hi * a.Wi * a.Cin * 2 < 2147483648.0;
}

template <typename T, int CIN, int COUT>
static void launch_conv_halo_c(const Exec& ex, const GemmArgs& a, int tx, int ty, int grid) {
  if (a.relu_in) hipLaunchKernelGGL((conv3x3_halo_kernel<T, CIN, COUT, true>), dim3(grid), dim3(576), 0, ex.stream, a, tx, ty);
  else hipLaunchKernelGGL((conv3x3_halo_kernel<T, CIN, COUT, false>), dim3(grid), dim3(576), 0, ex.stream, a, tx, ty);
}

template <typename T>
static void launch_conv_halo(const Exec& ex, const GemmArgs& a) {
  const int tx = cdiv(a.Wo, 32), ty = cdiv(a.Ho, 8);
  const long tiles = long(a.V) * tx * ty;
  const int grid = int(std::min<long>(tiles, GEMM_CUS));
  if (a.Cin == 64 && a.N == 64) launch_conv_halo_c<T, 64, 64>(ex, a, tx, ty, grid);
  else if (a.Cin == 64) launch_conv_halo_c<T, 64, 32>(ex, a, tx, ty, grid);
  else if (a.N == 64) launch_conv_halo_c<T, 32, 64>(ex, a, tx, ty, grid);
  else launch_conv_halo_c<T, 32, 32>(ex, a, tx, ty, grid);
  SPLAT_HIP(hipGetLastError());
}

// The 16-bit types (bf16, f16) share the tile configurations.
template <typename H>
static bool launch_h16_auto(const Exec& ex, const GemmArgs& a) {
  if (conv_halo_ok(a)) {
    launch_conv_halo<H>(ex, a);
    return false;
  }
  const BfCfg c = pick_bf16(a);
  int S = split_factor(a, c);
  if (S > 1 && !(ex.ws && ex.ws->ptr && ex.ws->cap >= split_bytes(a, S))) S = 1;
  // Convolutions whose Cin is a multiple of 32 but not of 64 (96-channel maps): 32-element
  // k-tiles keep them on the per-tap path for the tiles whose rows split into 16-row loads
  // (256x256 with a third stage, so that the epilogue slabs fit the ring)
  if (a.amode == A_CONV && a.Cin % 64 != 0 && a.Cin % 32 == 0 && a.ks * a.ks <= 32 && !a.hw3) {
    switch (c) {
      case CFG_128x64: return launch_mfma<H, 128, 64, 2, 2, 2, 32, 1, true>(ex, a, S);
      case CFG_256x256: return launch_mfma<H, 256, 256, 2, 4, 3, 32, 1, true>(ex, a, S);
      case CFG_256x128: return launch_mfma<H, 256, 128, 4, 2, 3, 32, 1, true>(ex, a, S);
      case CFG_128x128: return launch_mfma<H, 128, 128, 2, 2, 4, 32, 1, true>(ex, a, S);
      default: break;  // 320- and 192-row and 32-column tiles: the per-lane path
    }
  }
  switch (c) {
    case CFG_128x32: return launch_mfma<H, 128, 32, 4, 1, 2>(ex, a, S);
    case CFG_128x64: return launch_mfma<H, 128, 64, 2, 2, 2>(ex, a, S);
    // three A stages, two W stages (the whole 160 KB): 8192^3 990 -> 950 us, 8192x8192x2048 233 ->
    // 225 us; the C4 layer shapes (12-16 k-tiles a tile) unchanged
    case CFG_256x256: return launch_mfma<H, 256, 256, 2, 4, 2, 64, 1, false, 3>(ex, a, S);
    case CFG_256x128: return launch_mfma<H, 256, 128, 4, 2, 3>(ex, a, S);
    case CFG_320x256: return launch_mfma<H, 320, 256, 2, 4, 2>(ex, a, S);
    case CFG_320x128: return launch_mfma<H, 320, 128, 2, 4, 2>(ex, a, S);
    case CFG_192x128: return launch_mfma<H, 192, 128, 2, 4, 3>(ex, a, S);
    case CFG_192x128D: return launch_mfma<H, 192, 128, 2, 4, 2, 64, 2>(ex, a, S);
    default: return launch_mfma<H, 128, 128, 2, 2, 4>(ex, a, S);
  }
}

template <typename T, int BM, int BN, int WM, int WN>
static void launch_cfg(const Exec& ex, const GemmArgs& a) {
  dim3 grid(cdiv(a.M, BM), cdiv(a.N, BN));
  if (a.amode == A_ROWS)
    hipLaunchKernelGGL((gemm_kernel<T, BM, BN, WM, WN, A_ROWS>), grid, dim3(256), 0, ex.stream, a);
  else
    hipLaunchKernelGGL((gemm_kernel<T, BM, BN, WM, WN, A_CONV>), grid, dim3(256), 0, ex.stream, a);
  SPLAT_HIP(hipGetLastError());
}

// The MFMA path addresses its operands with 32-bit buffer offsets.
static bool mfma_path_ok(const GemmArgs& a) {
  const double es = a.dt == F32 ? 4 : 2;
  const double abytes = a.amode == A_ROWS ? double(a.M) * a.lda * es : double(a.V) * a.Hi * a.Wi * a.Cin * es;
  return abytes < 2147483648.0 && double(a.N) * a.ldw * es < 2147483648.0;
}

template <typename T>
static bool launch_typed(const Exec& ex, const GemmArgs& a) {
  if (mfma_path_ok(a)) {
    if constexpr (sizeof(T) == 2) return launch_h16_auto<T>(ex, a);
    else return launch_f32_auto(ex, a);
  }
  SPLAT_CHECK(a.hw3 == nullptr && a.ln_in == nullptr, BAD_ARGUMENT,
              "gemm: the fused head and the folded LayerNorm need the MFMA path");
  const long tiles128 = (long)cdiv(a.M, 128) * cdiv(a.N, 128);
  if (a.N <= 32) launch_cfg<T, 256, 32, 4, 1>(ex, a);
  else if (a.N <= 64) launch_cfg<T, 256, 64, 4, 1>(ex, a);
  else if (tiles128 >= 512) launch_cfg<T, 128, 128, 2, 2>(ex, a);
  else launch_cfg<T, 64, 128, 1, 4>(ex, a);
  return false;
}

void gemm(const Exec& ex, const GemmArgs& args) {
  GemmArgs a = args;
  a.epi_vec = epi_vec_ok(a, a.dt == F32 ? 4 : 2) ? 1 : 0;
  const int ke = a.dt == F32 ? 4 : 8;
  SPLAT_CHECK(a.M >= 0 && a.N > 0 && a.K > 0, BAD_ARGUMENT, "gemm: bad sizes");
  SPLAT_CHECK(a.K % ke == 0, BAD_ARGUMENT, "gemm: K must be a multiple of the 16-byte chunk");
  SPLAT_CHECK(a.ldw % 64 == 0 && a.ldw >= ((a.K + 63) / 64) * 64, BAD_ARGUMENT, "gemm: W must be padded to 64");
  SPLAT_CHECK((reinterpret_cast<uintptr_t>(a.A) & 15) == 0 && (reinterpret_cast<uintptr_t>(a.W) & 15) == 0,
              BAD_ARGUMENT, "gemm: operands must be 16-byte aligned");
  if (a.amode == A_ROWS) SPLAT_CHECK(a.lda % ke == 0 && a.lda >= a.K, BAD_ARGUMENT, "gemm: bad lda");
  else {
    SPLAT_CHECK(a.Cin % ke == 0 && a.K == a.ks * a.ks * a.Cin, BAD_ARGUMENT, "gemm: conv Cin/K");
    SPLAT_CHECK((long)a.V * a.Ho * a.Wo == a.M, BAD_ARGUMENT, "gemm: conv M != V*Ho*Wo");
  }
  if (a.store == STORE_CONVT)
    SPLAT_CHECK((long)a.ct_s * a.ct_s * a.ct_Cout == a.N && (long)a.V * a.ct_R * a.ct_C == a.M, BAD_ARGUMENT,
                "gemm: convT geometry");
  if (a.ln_in)
    SPLAT_CHECK(a.ln_c1 && a.ln_eps > 0.f && a.ln_parts > 0 && a.ln_parts <= 16 && a.amode == A_ROWS && !a.res &&
                    !a.gamma && !a.res2 && !a.addtab && !a.rm_P && !a.act_post && a.store == STORE_ROWS && a.epi_vec,
                BAD_ARGUMENT, "gemm: a folded LayerNorm needs plain aligned rows, a bias/activation epilogue and "
                              "at most 16 partials a row");
  if (a.glu)
    SPLAT_CHECK(a.ln_in && a.N % 16 == 0 && !a.qk_dim && a.act == ACT_NONE && a.ldc >= a.N / 2, BAD_ARGUMENT,
                "gemm: the SwiGLU gate needs a folded-LayerNorm w12 GEMM with interleaved rows");
  if (a.qk_dim)
    SPLAT_CHECK(a.ln_in && a.N == 3 * a.qk_dim && a.qk_dim % 64 == 0 && (a.qw == nullptr) == (a.qb == nullptr) &&
                    (a.kw == nullptr) == (a.kb == nullptr) && (!a.rope_cs || (a.rope_n > 0 && a.rope_cols > 0)),
                BAD_ARGUMENT, "gemm: qk-norm + RoPE need a folded-LayerNorm qkv GEMM");
  if (a.q_cols)
    SPLAT_CHECK(a.ln_in && a.q_cols % 8 == 0 && a.q_cols <= a.N && !a.glu, BAD_ARGUMENT,
                "gemm: the Q scale needs a folded-LayerNorm qkv GEMM");
  if (a.rope_cs && !a.rope_across && a.qk_dim)
    SPLAT_CHECK((a.rope_n - 1) / a.rope_cols + 1 < a.rope_npos && a.rope_cols + 1 <= a.rope_npos, BAD_ARGUMENT,
                "gemm: RoPE table too small");
  if (a.ln_out)
    SPLAT_CHECK((a.ln_group == 64 || a.ln_group == 128) && a.N % a.ln_group == 0 && a.out_f32 &&
                    a.store == STORE_ROWS && !a.rm_P && a.ldc % 4 == 0 && (reinterpret_cast<uintptr_t>(a.out) & 15) == 0 &&
                    (reinterpret_cast<uintptr_t>(a.ln_copy) & 15) == 0,
                BAD_ARGUMENT, "gemm: row statistics need fp32 rows and N a multiple of the group");
  if (ex.dry && ex.ws && a.M > 0 && mfma_path_ok(a))  // size the split-K partials of the real run
    ex.ws->need = std::max(ex.ws->need, split_bytes(a, split_factor(a, a.dt == F32 ? pick_f32(a) : pick_bf16(a))));
  if (ex.dry || a.M == 0) return;
  const double es = a.dt == F32 ? 4 : 2, mn = double(a.M) * a.N;
  const double abytes = a.amode == A_ROWS ? double(a.M) * a.K * es : double(a.V) * a.Hi * a.Wi * a.Cin * es;
  const double bytes = abytes + double(a.N) * a.K * es + mn * (a.out_f32 ? 4 : es) +
                       (a.res ? mn * (a.res_f32 ? 4 : es) : 0) + (a.res2 ? mn * (a.res2_f32 ? 4 : es) : 0);
  bool stats;
  {
    ProfScope ps(ex, a.amode == A_ROWS ? "gemm" : "conv_igemm", 2.0 * mn * a.K, bytes);
    stats = a.dt == F32 ? launch_typed<float>(ex, a) : a.dt == F16 ? launch_typed<f16>(ex, a) : launch_typed<bf16>(ex, a);
  }
  if (a.ln_out && !stats)  // this path's epilogue does not emit them
    ln_stats(ex, static_cast<const float*>(a.out), a.ldc, a.M, a.N, a.ln_group, a.ln_out, a.dt, a.ln_copy);
}

}  // namespace splat
