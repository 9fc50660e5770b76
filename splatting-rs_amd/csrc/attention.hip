// Flash attention for head dim 64 on the matrix cores (no mask, scale 1/8), used for the
// per-view (local) and the cross-view (global) blocks alike: a launch covers `seqs`
// sequences of L tokens each, every (sequence, head) independent.
//
// Each wave owns 32 queries. Scores are computed transposed, S^T = K Q^T, so that in the
// accumulator layout (lane l, register r -> row 8*(r/4) + 4*(l/32) + r%4, column l%32) a
// lane holds one query (column) and 16 keys per 32-key tile. That same register set is the
// B operand of O^T = V^T P^T with no data movement: the k-slot order of the P fragment is
// mirrored when reading V^T, which lives transposed in LDS. Softmax is online (running max
// and sum per query, base-2 exponent with the 1/8*log2(e) scale folded into one FMA); the
// row max needs one exchange between lanes l and l^32.
#include "kernels.h"

namespace splat {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

namespace {

template <typename T> struct AttnOps;
template <> struct AttnOps<bf16> {
  // O^T[d][q] += V^T[d][keys] P^T[keys][q] for the 32 keys of sub-tile kt2.
  __device__ static inline void pv(f32x16& o, const char* vrow, int kt2, int g, const f32x16& s) {
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const char* base = vrow + (kt2 * 32 + 16 * hh + 4 * g) * 2;
      uint2 lo = *reinterpret_cast<const uint2*>(base);
      uint2 hi = *reinterpret_cast<const uint2*>(base + 16);
      uint4 vf = make_uint4(lo.x, lo.y, hi.x, hi.y);
      uint4 pf;
      uint32_t* pw = reinterpret_cast<uint32_t*>(&pf);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        pw[i] = uint32_t(f2bf(s[8 * hh + 2 * i])) | (uint32_t(f2bf(s[8 * hh + 2 * i + 1])) << 16);
      o = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, vf), __builtin_bit_cast(bf16x8_t, pf),
                                                  o, 0, 0, 0);
    }
  }
  __device__ static inline void qk(f32x16& acc, const uint4& kf, const uint4& qf) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, kf), __builtin_bit_cast(bf16x8_t, qf),
                                                  acc, 0, 0, 0);
  }
  __device__ static inline void store4(void* dst, const float* v) {
    uint2 w;
    w.x = uint32_t(f2bf(v[0])) | (uint32_t(f2bf(v[1])) << 16);
    w.y = uint32_t(f2bf(v[2])) | (uint32_t(f2bf(v[3])) << 16);
    *reinterpret_cast<uint2*>(dst) = w;
  }
};
template <> struct AttnOps<float> {
  __device__ static inline void pv(f32x16& o, const char* vrow, int kt2, int g, const f32x16& s) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float4 vf = *reinterpret_cast<const float4*>(vrow + (kt2 * 32 + 8 * q + 4 * g) * 4);
      o = __builtin_amdgcn_mfma_f32_32x32x2f32(vf.x, s[4 * q + 0], o, 0, 0, 0);
      o = __builtin_amdgcn_mfma_f32_32x32x2f32(vf.y, s[4 * q + 1], o, 0, 0, 0);
      o = __builtin_amdgcn_mfma_f32_32x32x2f32(vf.z, s[4 * q + 2], o, 0, 0, 0);
      o = __builtin_amdgcn_mfma_f32_32x32x2f32(vf.w, s[4 * q + 3], o, 0, 0, 0);
    }
  }
  __device__ static inline void qk(f32x16& acc, const uint4& kf, const uint4& qf) {
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(kf.x), __uint_as_float(qf.x), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(kf.y), __uint_as_float(qf.y), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(kf.z), __uint_as_float(qf.z), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(kf.w), __uint_as_float(qf.w), acc, 0, 0, 0);
  }
  __device__ static inline void store4(void* dst, const float* v) {
    *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
  }
};

}  // namespace

constexpr int ATTN_WAVES = 4;

template <typename T>
__global__ void __launch_bounds__(ATTN_WAVES * 64) attn_kernel(const AttnArgs p, float c) {
  constexpr int ES = sizeof(T);
  constexpr int KE = 16 / ES;              // elements per 16-byte fragment
  constexpr int DSTEPS = 64 / (2 * KE);    // k-steps over the head dim (32 bytes each)
  constexpr int KROW = 64 * ES + 16;       // LDS bytes per K row
  constexpr int VROW = 64 * ES + (ES == 2 ? 8 : 16);  // LDS bytes per V^T row (64 keys)
  constexpr int CPR = 64 * ES / 16;        // 16-byte chunks per K row
  constexpr int NT = ATTN_WAVES * 64;
  constexpr int KCH = 64 * CPR / NT;       // K chunks per thread per tile
  __shared__ __attribute__((aligned(16))) char ks[2][64 * KROW];
  __shared__ __attribute__((aligned(16))) char vts[2][64 * VROW];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int h = blockIdx.y;
  const long base = (long)blockIdx.z * p.seq_stride;
  const long q0 = (long)blockIdx.x * (ATTN_WAVES * 32) + wave * 32;
  const T* Q = reinterpret_cast<const T*>(p.q) + h * 64;
  const T* K = reinterpret_cast<const T*>(p.k) + h * 64;
  const T* V = reinterpret_cast<const T*>(p.v) + h * 64;

  const long qrow = q0 + l32;
  const bool qok = qrow < p.L;
  uint4 qf[DSTEPS];
#pragma unroll
  for (int st = 0; st < DSTEPS; ++st)
    qf[st] = qok ? *reinterpret_cast<const uint4*>(Q + (base + qrow) * p.ld + st * 2 * KE + g * KE)
                 : make_uint4(0, 0, 0, 0);

  // tile loaders
  uint4 rk[KCH];
  uint4 rv[4];  // 4 keys x 4 head channels (bf16: low 8 bytes used)
  const int vkq = tid / 16, vdq = tid % 16;
  auto gload = [&](int t) {
    const long k0 = (long)t * 64;
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int cidx = tid + i * NT, row = cidx / CPR, col = cidx % CPR;
      rk[i] = (k0 + row < p.L) ? *reinterpret_cast<const uint4*>(K + (base + k0 + row) * p.ld + col * KE)
                               : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const long key = k0 + 4 * vkq + j;
      if (key < p.L) {
        const T* src = V + (base + key) * p.ld + 4 * vdq;
        if (ES == 2) {
          uint2 w = *reinterpret_cast<const uint2*>(src);
          rv[j] = make_uint4(w.x, w.y, 0, 0);
        } else {
          rv[j] = *reinterpret_cast<const uint4*>(src);
        }
      } else {
        rv[j] = make_uint4(0, 0, 0, 0);
      }
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int cidx = tid + i * NT, row = cidx / CPR, col = cidx % CPR;
      *reinterpret_cast<uint4*>(&ks[buf][row * KROW + col * 16]) = rk[i];
    }
    // transpose the 4x4 block: Vt[4*vdq + e][4*vkq + j] = V[4*vkq + j][4*vdq + e]
    if (ES == 2) {
      const uint16_t* e16[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) e16[j] = reinterpret_cast<const uint16_t*>(&rv[j]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        uint2 w;
        w.x = uint32_t(e16[0][e]) | (uint32_t(e16[1][e]) << 16);
        w.y = uint32_t(e16[2][e]) | (uint32_t(e16[3][e]) << 16);
        *reinterpret_cast<uint2*>(&vts[buf][(4 * vdq + e) * VROW + 4 * vkq * 2]) = w;
      }
    } else {
      const uint32_t* e32[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) e32[j] = reinterpret_cast<const uint32_t*>(&rv[j]);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        *reinterpret_cast<uint4*>(&vts[buf][(4 * vdq + e) * VROW + 4 * vkq * 4]) =
            make_uint4(e32[0][e], e32[1][e], e32[2][e], e32[3][e]);
    }
  };

  f32x16 o[2];
#pragma unroll
  for (int r = 0; r < 16; ++r) { o[0][r] = 0.f; o[1][r] = 0.f; }
  float m = -INFINITY, lsum = 0.f;

  const int ntiles = (p.L + 63) / 64;
  gload(0);
  sstore(0);
  __syncthreads();
  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    if (t + 1 < ntiles) gload(t + 1);
    f32x16 s[2];
#pragma unroll
    for (int kt2 = 0; kt2 < 2; ++kt2) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[kt2][r] = 0.f;
#pragma unroll
      for (int st = 0; st < DSTEPS; ++st) {
        uint4 kf = *reinterpret_cast<const uint4*>(&ks[buf][(kt2 * 32 + l32) * KROW + (2 * st + g) * 16]);
        AttnOps<T>::qk(s[kt2], kf, qf[st]);
      }
    }
    const long k0 = (long)t * 64;
    if (k0 + 64 > p.L) {
#pragma unroll
      for (int kt2 = 0; kt2 < 2; ++kt2)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (k0 + kt2 * 32 + 8 * (r >> 2) + 4 * g + (r & 3) >= p.L) s[kt2][r] = -INFINITY;
    }
    float mx = s[0][0];
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, fmaxf(s[0][r], s[1][r]));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float mnew = fmaxf(m, mx);
    const float alpha = exp2f((m - mnew) * c);
    const float mc = mnew * c;
    float ps = 0.f;
#pragma unroll
    for (int kt2 = 0; kt2 < 2; ++kt2)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float e = exp2f(fmaf(s[kt2][r], c, -mc));
        s[kt2][r] = e;
        ps += e;
      }
    lsum = lsum * alpha + ps;
    m = mnew;
#pragma unroll
    for (int r = 0; r < 16; ++r) { o[0][r] *= alpha; o[1][r] *= alpha; }
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) {
      const char* vrow = &vts[buf][(dt * 32 + l32) * VROW];
#pragma unroll
      for (int kt2 = 0; kt2 < 2; ++kt2) AttnOps<T>::pv(o[dt], vrow, kt2, g, s[kt2]);
    }
    if (t + 1 < ntiles) sstore(buf ^ 1);
    __syncthreads();
  }

  const float ltot = lsum + __shfl_xor(lsum, 32);
  const float inv = 1.f / ltot;
  if (qok) {
    T* O = reinterpret_cast<T*>(p.o) + (base + qrow) * p.ldo + h * 64;
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = o[dt][4 * q4 + e] * inv;
        AttnOps<T>::store4(O + dt * 32 + 8 * q4 + 4 * g, v);
      }
  }
}

void attention(const Exec& ex, const AttnArgs& a) {
  const int ke = a.dt == F32 ? 4 : 8;
  SPLAT_CHECK(a.L > 0 && a.heads > 0 && a.seqs > 0, BAD_ARGUMENT, "attention: bad sizes");
  SPLAT_CHECK(a.ld % ke == 0 && a.ldo % 4 == 0 && a.ld >= (long)a.heads * 64, BAD_ARGUMENT, "attention: strides");
  SPLAT_CHECK(a.seqs == 1 || a.seq_stride >= a.L, BAD_ARGUMENT, "attention: overlapping sequences");
  if (ex.dry) return;
  const double rows = double(a.seqs) * a.L * a.heads;
  ProfScope ps(ex, "attention", 4.0 * rows * a.L * 64, 4.0 * rows * 64 * (a.dt == F32 ? 4 : 2));
  dim3 grid(cdiv(a.L, ATTN_WAVES * 32), a.heads, a.seqs);
  const float c = 0.125f * 1.4426950408889634f;
  if (a.dt == F32) hipLaunchKernelGGL(attn_kernel<float>, grid, dim3(ATTN_WAVES * 64), 0, ex.stream, a, c);
  else hipLaunchKernelGGL(attn_kernel<bf16>, grid, dim3(ATTN_WAVES * 64), 0, ex.stream, a, c);
  SPLAT_HIP(hipGetLastError());
}

}  // namespace splat
