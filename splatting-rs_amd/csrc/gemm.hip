// MFMA GEMM with fused prologue (implicit-im2col conv, ReLU-on-load) and epilogue (bias,
// GELU/ReLU, table add, LayerScale, up to two residuals, row remap, transposed-conv scatter).
//
// Both operands are "K-contiguous": A [M, K] (or an implicit im2col of an NHWC map) and
// W [N, K] (PyTorch Linear / conv weight order). A k-tile is 128 bytes of K per row (64 bf16
// or 32 fp32). Each lane feeds the matrix core a 16-byte fragment of one row: lanes 0-31 the
// first 16 bytes of a 32-byte k-step, lanes 32-63 the second; A and W use the same k order,
// so the sum over k is exact whatever order the hardware walks the fragment in.
//   bf16: one v_mfma_f32_32x32x16_bf16 per k-step;
//   fp32: four v_mfma_f32_32x32x2_f32, one per float of the fragment.
// Accumulator layout (32x32 MFMA): lane l, register r -> row 8*(r/4) + 4*(l/32) + r%4,
// column l%32.
#include "kernels.h"

namespace splat {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

template <typename T> struct Mfma;
template <> struct Mfma<bf16> {
  __device__ static inline void mma(f32x16& acc, const uint4& a, const uint4& b) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                  acc, 0, 0, 0);
  }
  __device__ static inline uint4 relu(uint4 v) {
    uint32_t* w = reinterpret_cast<uint32_t*>(&v);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t x = w[i];
      uint32_t lo = (x & 0x8000u) ? 0u : (x & 0xffffu);
      uint32_t hi = (x & 0x80000000u) ? 0u : (x & 0xffff0000u);
      w[i] = lo | hi;
    }
    return v;
  }
};
template <> struct Mfma<float> {
  __device__ static inline void mma(f32x16& acc, const uint4& a, const uint4& b) {
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.x), __uint_as_float(b.x), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.y), __uint_as_float(b.y), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.z), __uint_as_float(b.z), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.w), __uint_as_float(b.w), acc, 0, 0, 0);
  }
  __device__ static inline uint4 relu(uint4 v) {
    uint32_t* w = reinterpret_cast<uint32_t*>(&v);
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = (w[i] & 0x80000000u) ? 0u : w[i];
    return v;
  }
};

__device__ inline float gelu_erf(float x) { return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f)); }

// A residual is fp32 when flagged, else stored in the kernel's own dtype T.
template <typename T>
__device__ inline float load_res(const void* p, long i, int f32) {
  if (f32 || sizeof(T) == 4) return reinterpret_cast<const float*>(p)[i];
  return bf2f(reinterpret_cast<const bf16*>(p)[i]);
}

constexpr int LDS_ROW = 144;  // bytes per tile row: 128 bytes of K + 16 bytes against bank conflicts

template <typename T, int BM, int BN, int WM, int WN, int AMODE>
__global__ void __launch_bounds__(256) gemm_kernel(const GemmArgs p) {
  constexpr int KE = 16 / sizeof(T);        // elements per 16-byte chunk
  constexpr int BK = 8 * KE;                // elements per k-tile
  constexpr int TM = BM / WM / 32, TN = BN / WN / 32;
  constexpr int ACH = BM / 32, BCH = BN / 32;  // 16-byte chunks per thread per tile
  __shared__ __attribute__((aligned(16))) char smem[2 * (BM + BN) * LDS_ROW];

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

  // ---- epilogue
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const long n = n0 + wn * (BN / WN) + j * 32 + l32;
    if (n >= p.N) continue;
    const float bias = p.bias ? p.bias[n] : 0.f;
    const float gam = p.gamma ? p.gamma[n] : 1.f;
    long ct_t = 0, ct_co = 0, ct_dy = 0, ct_dx = 0;
    if (p.store == STORE_CONVT) {
      ct_t = n / p.ct_Cout;
      ct_co = n - ct_t * p.ct_Cout;
      ct_dy = ct_t / p.ct_s;
      ct_dx = ct_t - ct_dy * p.ct_s;
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const long m = m0 + wm * (BM / WM) + i * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
        if (m >= p.M) continue;
        float v = acc[i][j][r] + bias;
        if (p.act == ACT_RELU) v = fmaxf(v, 0.f);
        else if (p.act == ACT_GELU) v = gelu_erf(v);
        if (p.addtab) v += p.addtab[(m % p.addtab_period) * p.N + n];
        v *= gam;
        long row = p.rm_P ? (m / p.rm_P) * p.rm_n + p.rm_off + m % p.rm_P : m;
        if (p.res) v += load_res<T>(p.res, row * p.ldres + n, p.res_f32);
        if (p.res2) v += load_res<T>(p.res2, row * p.ldres2 + n, p.res2_f32);
        long idx;
        if (p.store == STORE_CONVT) {
          const long hw = (long)p.ct_R * p.ct_C;
          const long vv = m / hw, rem = m - vv * hw;
          const long rr = rem / p.ct_C, cc = rem - rr * p.ct_C;
          const long Wout = (long)p.ct_C * p.ct_s;
          idx = ((vv * p.ct_R * p.ct_s + rr * p.ct_s + ct_dy) * Wout + cc * p.ct_s + ct_dx) * p.ct_Cout + ct_co;
        } else {
          idx = row * p.ldc + n;
        }
        if (p.out_f32) reinterpret_cast<float*>(p.out)[idx] = v;
        else reinterpret_cast<T*>(p.out)[idx] = from_f<T>(v);
      }
    }
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

template <typename T>
static void launch_typed(const Exec& ex, const GemmArgs& a) {
  const long tiles128 = (long)cdiv(a.M, 128) * cdiv(a.N, 128);
  if (a.N <= 32) launch_cfg<T, 256, 32, 4, 1>(ex, a);
  else if (a.N <= 64) launch_cfg<T, 256, 64, 4, 1>(ex, a);
  else if (tiles128 >= 512) launch_cfg<T, 128, 128, 2, 2>(ex, a);
  else launch_cfg<T, 64, 128, 1, 4>(ex, a);
}

void gemm(const Exec& ex, const GemmArgs& a) {
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
  if (ex.dry || a.M == 0) return;
  const double es = a.dt == F32 ? 4 : 2, mn = double(a.M) * a.N;
  const double abytes = a.amode == A_ROWS ? double(a.M) * a.K * es : double(a.V) * a.Hi * a.Wi * a.Cin * es;
  const double bytes = abytes + double(a.N) * a.K * es + mn * (a.out_f32 ? 4 : es) +
                       (a.res ? mn * (a.res_f32 ? 4 : es) : 0) + (a.res2 ? mn * (a.res2_f32 ? 4 : es) : 0);
  ProfScope ps(ex, a.amode == A_ROWS ? "gemm" : "conv_igemm", 2.0 * mn * a.K, bytes);
  if (a.dt == F32) launch_typed<float>(ex, a);
  else launch_typed<bf16>(ex, a);
}

}  // namespace splat
