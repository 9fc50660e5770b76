// Flash attention for head dim 64 on the matrix cores (no mask, scale 1/8), used for the
// per-view (local) and the cross-view (global) blocks alike: a launch covers `seqs`
// sequences of L tokens each, every (sequence, head) independent.
//
// Each wave owns 32 queries. Scores are computed transposed, S^T = K Q^T, so that in the
// accumulator layout (lane l, register r -> row 8*(r/4) + 4*(l/32) + r%4, column l%32) a
// lane holds one query (column) and 16 keys per 32-key tile. That same register set is the
// B operand of O^T = V^T P^T with no data movement: the k-slot order of the P fragment is
// mirrored when reading V^T, which lives transposed in LDS. Softmax is online: base-2
// exponents, the running sum per query, and (generic kernel below) a running max whose row
// reduction needs one exchange between lanes l and l^32.
#include "kernels.h"

#include <algorithm>
#include <cmath>
#include <functional>
#include <mutex>
#include <type_traits>

namespace splat {

// Device-resident scratch for the key-slice partials of attention launches that must not
// allocate (splat_kernel_attention_noalloc): one copy per GPU, held until the process ends.
// Host code never passes `scratch` itself to a kernel (on the host the name is only a stand-in
// for the symbol): attention_scratch() looks up each device's address once, with that device
// current, and callers use that address.
static __device__ __align__(256) char scratch[ATTN_SCRATCH_BYTES];

namespace {
std::mutex g_scratch_mu;
void* g_scratch_addr[ATTN_SCRATCH_DEVICES] = {};
// Per device: the event recorded after the last eager launch that used the scratch, and the lock
// that orders the wait / launch / record sequences of concurrent callers.
hipEvent_t g_scratch_done[ATTN_SCRATCH_DEVICES] = {};
bool g_scratch_recorded[ATTN_SCRATCH_DEVICES] = {};
std::mutex g_scratch_order[ATTN_SCRATCH_DEVICES];
}  // namespace

void* attention_scratch(int device) {
  SPLAT_CHECK(device >= 0 && device < ATTN_SCRATCH_DEVICES, BAD_ARGUMENT, "attention scratch: device index");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_addr[device]) {
    int cur = -1;
    SPLAT_HIP(hipGetDevice(&cur));
    SPLAT_CHECK(cur == device, BAD_ARGUMENT, "attention scratch: the device must be current");
    void* p = nullptr;
    SPLAT_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    SPLAT_CHECK(p != nullptr, HIP_ERROR, "attention scratch: no device address");
    SPLAT_HIP(hipEventCreateWithFlags(&g_scratch_done[device], hipEventDisableTiming));
    g_scratch_addr[device] = p;
  }
  return g_scratch_addr[device];
}

void attention_scratch_ordered(int device, hipStream_t stream, const std::function<void()>& launch) {
  SPLAT_CHECK(device >= 0 && device < ATTN_SCRATCH_DEVICES && g_scratch_done[device], BAD_ARGUMENT,
              "attention scratch: not set up on this device");
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  SPLAT_HIP(hipStreamIsCapturing(stream, &cap));
  if (cap != hipStreamCaptureStatusNone) {  // a captured launch: the caller's graph orders it
    launch();
    return;
  }
  std::lock_guard<std::mutex> lock(g_scratch_order[device]);
  if (g_scratch_recorded[device]) SPLAT_HIP(hipStreamWaitEvent(stream, g_scratch_done[device], 0));
  launch();
  SPLAT_HIP(hipEventRecord(g_scratch_done[device], stream));
  g_scratch_recorded[device] = true;
}

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

namespace {

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

// 32x32x16 product of 16-bit operand fragments (8 values a lane) of storage type H
template <typename H> __device__ inline f32x16 mma16(const uint4& a, const uint4& b, const f32x16& c);
template <> __device__ inline f32x16 mma16<bf16>(const uint4& a, const uint4& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
template <> __device__ inline f32x16 mma16<f16>(const uint4& a, const uint4& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}
// acc + the two values of a packed pair (one v_dot2 against a pair of ones)
template <typename H> __device__ inline float add_pair(uint32_t pair, float acc);
template <> __device__ inline float add_pair<bf16>(uint32_t pair, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, pair), __builtin_bit_cast(bf16x2_t, 0x3f803f80u), acc,
                                         false);
}
template <> __device__ inline float add_pair<f16>(uint32_t pair, float acc) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, pair), __builtin_bit_cast(f16x2_t, 0x3c003c00u), acc, false);
}

template <typename T> struct AttnOps;
template <typename H> struct AttnOps16 {
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
        pw[i] = pack2<H>(s[8 * hh + 2 * i], s[8 * hh + 2 * i + 1]);
      o = mma16<H>(vf, pf, o);
    }
  }
  __device__ static inline void qk(f32x16& acc, const uint4& kf, const uint4& qf) { acc = mma16<H>(kf, qf, acc); }
  __device__ static inline void store4(void* dst, const float* v) {
    uint2 w;
    w.x = pack2<H>(v[0], v[1]);
    w.y = pack2<H>(v[2], v[3]);
    *reinterpret_cast<uint2*>(dst) = w;
  }
};
template <> struct AttnOps<bf16> : AttnOps16<bf16> {};
template <> struct AttnOps<f16> : AttnOps16<f16> {};
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
constexpr int ATTN_MAX_SPLITS = 8;  // key slices a launch may use (attn_combine_kernel unrolls over them)

// SPLIT: the block covers key tiles [split * tps, (split + 1) * tps) and writes its unnormalised
// O and (max, sum) to p.part for attn_combine_kernel, as the bf16 kernel below does.
template <typename T, bool SPLIT>
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
  const int nq = (p.L + ATTN_WAVES * 32 - 1) / (ATTN_WAVES * 32);
  const int qb = SPLIT ? int(blockIdx.x) % nq : int(blockIdx.x), split = SPLIT ? int(blockIdx.x) / nq : 0;
  const long q0 = (long)qb * (ATTN_WAVES * 32) + wave * 32;
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
  const int t0 = SPLIT ? split * p.tps : 0, t1 = SPLIT ? min(ntiles, t0 + p.tps) : ntiles;
  gload(t0);
  sstore(0);
  __syncthreads();
  for (int t = t0; t < t1; ++t) {
    const int buf = (t - t0) & 1;
    if (t + 1 < t1) gload(t + 1);
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
    if (t + 1 < t1) sstore(buf ^ 1);
    __syncthreads();
  }

  const float ltot = lsum + __shfl_xor(lsum, 32);
  if constexpr (SPLIT) {
    if (qok) {
      const long rows = long(p.seqs) * p.L, row = long(blockIdx.z) * p.L + qrow;  // dense slice rows
      float* O = p.part + (long(split) * rows + row) * (long(p.heads) * 64) + h * 64;
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4)
          *reinterpret_cast<float4*>(O + dt * 32 + 8 * q4 + 4 * g) =
              make_float4(o[dt][4 * q4], o[dt][4 * q4 + 1], o[dt][4 * q4 + 2], o[dt][4 * q4 + 3]);
      if (g == 0) {  // the max in exp2 units, as the merge expects
        float* ml = p.part + long(p.nsplit) * rows * p.heads * 64 + ((long(split) * rows + row) * p.heads + h) * 2;
        *reinterpret_cast<float2*>(ml) = make_float2(m * c, ltot);
      }
    }
    return;
  }
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

// ---------------------------------------------------------------------------------------
// bf16 main path. Each wave owns QT*32 queries, so every K and V^T fragment read from LDS
// feeds QT matrix-core ops. K and V tiles stream straight into LDS, row-major as they lie in
// memory (buffer_load_dwordx4 ... lds, rows of 128 bytes = 64 head channels, XOR-swizzled by
// 16-byte chunk). The V^T operand of O^T = V^T P^T is read with ds_read_b64_tr_b16, which
// transposes 16-bit elements within each group of 16 lanes: no V pass through registers and no
// VALU transpose (C4 global attention 239 -> 213 us). Rows past the sequence read as zero
// (buffer range check) and are masked to -inf only in the last tile.
// Softmax: Q comes times log2(e)/8 (from the qkv GEMM's epilogue, or scaled here once per wave),
// so each score out of the matrix core is already the base-2 exponent s of its weight. The
// plain pass takes the weights as 2^s against a fixed reference 0: per score one v_exp_f32, a
// pack to bf16 and half a dot2 for the sum, no row maximum and no rescaling (C4 attention
// -10%, C5 global -14% against a running maximum). A query whose final sum lies outside
// [2^-64, 2^64] (logits beyond about +-44, or NaN) sends its block through a second, safe
// pass that keeps a per-query reference following the running maximum, moved only when a
// tile's maximum passes it by more than 8: O and the sum always share the reference, so both
// passes are exact up to rounding.

typedef int int32x4_t __attribute__((ext_vector_type(4)));
typedef const __attribute__((address_space(3))) char* lds_cptr_a;

namespace {

__device__ inline int32x4_t make_rsrc_a(const void* p, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  int32x4_t r;
  r[0] = __builtin_amdgcn_readfirstlane(int(uint32_t(a)));
  r[1] = __builtin_amdgcn_readfirstlane(int(uint32_t(a >> 32)));
  r[2] = __builtin_amdgcn_readfirstlane(int(bytes));
  r[3] = 0x00020000;
  return r;
}

// 16 bytes per lane from rsrc at voffset + soffset into LDS at lds + 16 * lane. A voffset of
// 0x80000000 reads zeros whatever soffset holds: every valid voffset + soffset lies inside the
// buffer (below 2^31), so the range check, with or without soffset, rejects only that one.
__device__ inline void load_lds_a(const int32x4_t& rsrc, uint32_t voffset, uint32_t soffset, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(__builtin_amdgcn_readfirstlane(int(lds))),
               "v"(voffset), "s"(rsrc), "s"(__builtin_amdgcn_readfirstlane(int(soffset)))
               : "memory");
}

__device__ inline float max3f(float a, float b, float c) { return fmaxf(fmaxf(a, b), c); }

template <int N> __device__ inline void wait_vm() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }

}  // namespace

// SPLIT: the block covers key tiles [split * tps, (split + 1) * tps) of its sequence and writes
// its unnormalised O and (reference, sum) to p.part; attn_combine_kernel merges the slices.
// H: the 16-bit storage type of Q, K, V and O (bf16 or f16).
template <int WAVES, int QT, bool SPLIT, typename H = bf16>
__global__ void __launch_bounds__(WAVES * 64, QT == 1 ? 4 : 2) attn_bf16_kernel(const AttnArgs p, float c) {
  constexpr int KBYTES = 64 * 128;            // K or V tile: 64 keys x 128 bytes, swizzled, unpadded
  constexpr int KL = 8 / WAVES;               // load instructions per wave per K (or V) tile
  static_assert(WAVES == 2 || WAVES == 4, "the load swizzles assume an even number of waves");
  // LDS: two K tiles, then two V tiles. K and V of tile t+1 are requested when tile t starts.
  // A third stage measured slower (C4 global 224 vs 207 us): it costs occupancy, and the loop
  // is bound by its VALU work, not by load latency.
  __shared__ __attribute__((aligned(1024))) char smem[4 * KBYTES];

  // the wave index is uniform, so every LDS destination of the DMA loads is scalar arithmetic
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, l32 = lane & 31;
  const int L = p.L;
  // 1D grid over (query block, head, sequence), query blocks fastest; the query blocks of one
  // head, which all stream the same K and V, run on one XCD.
  // (query block, slice) fastest, so that the blocks streaming one slice of one head's K and V
  // run on one XCD
  const int nq = (L + WAVES * QT * 32 - 1) / (WAVES * QT * 32);
  const int ns = SPLIT ? p.nsplit : 1;
  int qb, split, h, sq;
  bool whole = !SPLIT;  // the block covers every key tile and writes the output itself
  if (SPLIT && p.whole > 0) {
    // Tail split: (query block, head, sequence) units t < p.whole run whole, the rest in ns key
    // slices; each group is dealt to the XCDs on its own (p.whole is a multiple of 8)
    const int b = blockIdx.x;
    int t;
    if (b < p.whole) {
      t = xcd_contiguous(b, p.whole);
      split = 0;
      whole = true;
    } else {
      const int r = xcd_contiguous(b - p.whole, (nq * p.heads * p.seqs - p.whole) * ns);
      t = p.whole + r / ns;
      split = r % ns;
    }
    qb = t % nq;
    h = (t / nq) % p.heads;
    sq = t / (nq * p.heads);
  } else {
    const int id = xcd_contiguous(blockIdx.x, nq * ns * p.heads * p.seqs);
    qb = id % nq;
    split = (id / nq) % ns;
    h = (id / (nq * ns)) % p.heads;
    sq = id / (nq * ns * p.heads);
  }
  const long base = long(sq) * p.seq_stride;
  const bf16* Q = reinterpret_cast<const bf16*>(p.q) + h * 64;
  const bf16* V = reinterpret_cast<const bf16*>(p.v) + h * 64;
  const int q0 = (qb * WAVES + wave) * (QT * 32);
  // A wave whose queries all lie past the sequence (the last query block of a 1037-token view
  // has 13) still loads its share of every K/V tile and meets every barrier, but computes
  // nothing: the other waves on its SIMD get the matrix core and the VALU.
  const bool active = __builtin_amdgcn_readfirstlane(q0) < L;

  // Q times c = log2(e)/8, rounded to H once per wave: the products K Q^T are then the
  // softmax exponents in base 2, with no per-score scaling.
  uint4 qf[QT][4];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int qrow = q0 + qt * 32 + l32;
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const uint4 raw = qrow < L ? *reinterpret_cast<const uint4*>(Q + (base + qrow) * p.ld + st * 16 + g * 8)
                                 : make_uint4(0, 0, 0, 0);
      uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
      for (int i = 0; i < 4; ++i)
        w[i] = pack2<H>(u16f<H>(w[i]) * c, u16f<H>(w[i] >> 16) * c);
      qf[qt][st] = make_uint4(w[0], w[1], w[2], w[3]);
    }
  }

  // K and V rows: sequence row s -> byte offset within the buffer that starts at the
  // sequence's row 0. Lane offsets within a tile are fixed; the tile's t * 64 rows go in the
  // scalar offset, and only a tile that reaches past L checks its rows.
  const bf16* Kseq = reinterpret_cast<const bf16*>(p.k) + base * p.ld + h * 64;
  const int32x4_t rk = make_rsrc_a(Kseq, uint32_t(long(L) * p.ld * 2));
  // V rows: chunk c of row r in slot c ^ (2 * (r & 3)), so that the four consecutive rows one
  // 16-lane group of a transposed read touches sit on four different 32-byte bank groups.
  const bf16* Vseq = V + base * p.ld;
  const int32x4_t rv = make_rsrc_a(Vseq, uint32_t(long(L) * p.ld * 2));
  const int lrow = lane >> 3;
  const int kc = (lane & 7) ^ ((4 * (wave & 1) + (lrow >> 1)) & 7);
  const int vc = (lane & 7) ^ ((lrow & 3) << 1);
  const uint32_t tile_bytes = uint32_t(64 * p.ld * 2);
  int lrw[KL];
  uint32_t koff[KL], voff[KL];
#pragma unroll
  for (int i = 0; i < KL; ++i) {
    lrw[i] = (i * WAVES + wave) * 8 + lrow;
    koff[i] = uint32_t(lrw[i] * p.ld * 2 + kc * 16);
    voff[i] = uint32_t(lrw[i] * p.ld * 2 + vc * 16);
  }
  const uint32_t lds0 = uint32_t(reinterpret_cast<uintptr_t>((lds_cptr_a)smem));
  // K and V of tile t into ring slot B (compile time: the LDS destinations are constants)
  auto issue = [&](int t, auto bufc) {
    constexpr int B = decltype(bufc)::value;
    const uint32_t so = uint32_t(t) * tile_bytes;
    if (t * 64 + 64 <= L) {
#pragma unroll
      for (int i = 0; i < KL; ++i) {
        load_lds_a(rk, koff[i], so, lds0 + B * KBYTES + (i * WAVES + wave) * 1024);
        load_lds_a(rv, voff[i], so, lds0 + (2 + B) * KBYTES + (i * WAVES + wave) * 1024);
      }
    } else {
#pragma unroll
      for (int i = 0; i < KL; ++i) {
        const bool in = t * 64 + lrw[i] < L;
        load_lds_a(rk, in ? koff[i] : 0x80000000u, so, lds0 + B * KBYTES + (i * WAVES + wave) * 1024);
        load_lds_a(rv, in ? voff[i] : 0x80000000u, so, lds0 + (2 + B) * KBYTES + (i * WAVES + wave) * 1024);
      }
    }
  };
  // A operand of O^T[d][q] += V^T[d][keys] P^T[keys][q] for keys kt2*32 + 16*hh + (0..31): lane
  // l supplies d = dt*32 + l%32 and, in the k order of the P fragment, keys kA..kA+3 and
  // kA+8..kA+11 with kA = 16*hh + 4*(l/32). ds_read_b64_tr_b16 hands output lane i of a
  // 16-lane group element i of the 16 consecutive elements that source lanes 4j..4j+3 of the
  // group read, as its element j. So source lane s of group G reads row kA(G) + j (j = (s/4)%4)
  // at head channels dt*32 + 16*(G&1) + 4*(s%4): group G holds d = dt*32 + 16*(G&1) + (0..15)
  // and k-half G>>1.
  // vbase[dt] is lane l's byte offset for head channels dt*32.. in rows 0..15 of a V tile; the
  // 16-row groups kt2*32 + 16*hh add constants. It is recomputed in every tile from a copy of
  // the lane index the compiler cannot hoist: kept across the loop it would be spilled.
  auto vbases = [&](int (&vbase)[2]) {
    int ln;
    asm volatile("v_mov_b32 %0, %1" : "=v"(ln) : "v"(lane));
    const int G = ln >> 4, vj = (ln >> 2) & 3, vcc = ln & 3;
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
      vbase[dt] = (4 * (G >> 1) + vj) * 128 + (((4 * dt + 2 * (G & 1) + (vcc >> 1)) ^ (vj << 1)) * 16) + (vcc & 1) * 8;
  };
  auto vfrag = [&](const char* vt, const int (&vbase)[2], int kt2, int hh, int dt) {
    typedef short v4s __attribute__((ext_vector_type(4)));
    uint32_t w[4];
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const v4s r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)((
          lds_cptr_a)(vt + (kt2 * 32 + 16 * hh + 8 * half) * 128 + vbase[dt])));
      const uint2 u = __builtin_bit_cast(uint2, r);
      w[2 * half] = u.x;
      w[2 * half + 1] = u.y;
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
  };

  f32x16 o[QT][2];
  float mref[QT], lsum[QT];
  const int sw = (l32 >> 1) & 7;

  // One 64-key tile. Q arrives times log2(e)/8, so s = K Q^T is the base-2 exponent of each
  // key's weight. The plain pass (SAFE false) takes the weights as 2^s against a fixed
  // reference 0: no row maximum and no rescaling. The safe pass keeps a reference per query
  // that follows the running maximum, moved (and O and the sum rescaled) only when a tile's
  // maximum passes it by more than 8, so the weights stay below 2^8.
  auto tile = [&](int t, auto bufc, auto masked_t, auto safe_t) {
    constexpr bool masked = decltype(masked_t)::value, safe = decltype(safe_t)::value;
    constexpr int B = decltype(bufc)::value;
    const char* kb = smem + B * KBYTES;
    const char* vt = smem + (2 + B) * KBYTES;
    f32x16 s[QT][2];
    const f32x16 zero = {};
    // Wave priority 1 while issuing matrix-core work, 0 for the softmax: of the waves sharing a
    // SIMD (other blocks), one about to issue MFMAs goes first, so another's exponentials run
    // under its matrix-core time (C4 13.99 -> 13.87 ms, C5 64.3 -> 63.4 ms, A/B).
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int kt2 = 0; kt2 < 2; ++kt2)
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const uint4 kf = *reinterpret_cast<const uint4*>(kb + (kt2 * 32 + l32) * 128 + ((2 * st + g) ^ sw) * 16);
#pragma unroll
        for (int qt = 0; qt < QT; ++qt)  // the first k-step starts from a zero accumulator operand
          s[qt][kt2] = mma16<H>(kf, qf[qt][st], st == 0 ? zero : s[qt][kt2]);
      }
    __builtin_amdgcn_s_setprio(0);
    if constexpr (masked) {  // the peeled last tile only
      const int k0 = t * 64;
#pragma unroll
      for (int qt = 0; qt < QT; ++qt)
#pragma unroll
        for (int kt2 = 0; kt2 < 2; ++kt2)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (k0 + kt2 * 32 + 8 * (r >> 2) + 4 * g + (r & 3) >= L) s[qt][kt2][r] = -INFINITY;
    }
    if constexpr (safe) {
      bool grow = false;
      float mnew[QT];
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        // 32 exponents -> 1 with three-input maxima (v_max3_f32): 10 + 4 + 2 instructions
        float a[12];
#pragma unroll
        for (int i = 0; i < 5; ++i) {
          a[i] = max3f(s[qt][0][3 * i], s[qt][0][3 * i + 1], s[qt][0][3 * i + 2]);
          a[5 + i] = max3f(s[qt][1][3 * i], s[qt][1][3 * i + 1], s[qt][1][3 * i + 2]);
        }
        a[10] = s[qt][0][15];
        a[11] = s[qt][1][15];
        const float b0 = max3f(a[0], a[1], a[2]), b1 = max3f(a[3], a[4], a[5]), b2 = max3f(a[6], a[7], a[8]),
                    b3 = max3f(a[9], a[10], a[11]);
        float mx = fmaxf(max3f(b0, b1, b2), b3);
        // the other half of the query's keys sits in lane l ^ 32: one v_permlane32_swap gives
        // every lane both halves (a ds_bpermute costs an LDS round trip)
        const auto sw2 = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
        mx = fmaxf(__uint_as_float(sw2[0]), __uint_as_float(sw2[1]));
        mnew[qt] = mx > mref[qt] + 8.f ? mx : mref[qt];
        grow |= mnew[qt] != mref[qt];
      }
      if (__builtin_amdgcn_ballot_w64(grow)) {
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          const float alpha = __builtin_amdgcn_exp2f(mref[qt] - mnew[qt]);
          lsum[qt] *= alpha;
#pragma unroll
          for (int r = 0; r < 16; ++r) { o[qt][0][r] *= alpha; o[qt][1][r] *= alpha; }
          mref[qt] = mnew[qt];
        }
      }
#pragma unroll
      for (int qt = 0; qt < QT; ++qt)
#pragma unroll
        for (int kt2 = 0; kt2 < 2; ++kt2)
#pragma unroll
          for (int r = 0; r < 16; ++r) s[qt][kt2][r] = __builtin_amdgcn_exp2f(s[qt][kt2][r] - mref[qt]);
    } else {
#pragma unroll
      for (int qt = 0; qt < QT; ++qt)
#pragma unroll
        for (int kt2 = 0; kt2 < 2; ++kt2)
#pragma unroll
          for (int r = 0; r < 16; ++r) s[qt][kt2][r] = __builtin_amdgcn_exp2f(s[qt][kt2][r]);
    }
    int vbase[2];
    vbases(vbase);
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) {
#pragma unroll
      for (int kt2 = 0; kt2 < 2; ++kt2)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const uint4 vf = vfrag(vt, vbase, kt2, hh, dt);
#pragma unroll
          for (int qt = 0; qt < QT; ++qt) {
            uint4 pf;
            uint32_t* pw = reinterpret_cast<uint32_t*>(&pf);
#pragma unroll
            for (int i = 0; i < 4; ++i)
              pw[i] = pack2<H>(s[qt][kt2][8 * hh + 2 * i], s[qt][kt2][8 * hh + 2 * i + 1]);
            o[qt][dt] = mma16<H>(vf, pf, o[qt][dt]);
            if (dt == 0) {  // the running sum of the rounded P the matrix cores use: one dot2 per pair
#pragma unroll
              for (int i = 0; i < 4; ++i) lsum[qt] = add_pair<H>(pw[i], lsum[qt]);
            }
          }
        }
    }
    __builtin_amdgcn_s_setprio(0);
  };

  const int ntiles = (L + 63) / 64;
  const int t0 = whole ? 0 : split * p.tps, t1 = whole ? ntiles : min(ntiles, t0 + p.tps);
  const std::integral_constant<int, 0> R0;
  const std::integral_constant<int, 1> R1;
  // One pass over the slice's key tiles. Every tile but the last runs without the key mask (a
  // runtime flag inside one loop body was turned into selects that ran on every tile: ~100
  // VALU instructions per 64-key tile). Tile t sits in ring slot (t - t0) & 1; the loop is
  // unrolled by two so that the slot, and with it every LDS address, is a compile-time constant.
  auto pass = [&](auto safe_t) {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      mref[qt] = decltype(safe_t)::value ? -INFINITY : 0.f;
      lsum[qt] = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) { o[qt][0][r] = 0.f; o[qt][1][r] = 0.f; }
    }
    issue(t0, R0);
    wait_vm<0>();
    __syncthreads();
    auto step = [&](int t, auto bufc) {
      constexpr int B = decltype(bufc)::value;
      // slot B ^ 1 held tile t-1, which every wave finished before the last barrier
      issue(t + 1, std::integral_constant<int, B ^ 1>{});
      if (active) tile(t, bufc, std::false_type{}, safe_t);
      wait_vm<0>();  // this wave's share of tile t+1
      __syncthreads();
    };
    int t = t0;
    for (; t + 2 < t1; t += 2) {
      step(t, R0);
      step(t + 1, R1);
    }
    if (t + 1 < t1) step(t++, R0);
    // the slice's last tile, with the key mask (a no-op unless it holds the sequence's ragged
    // end): one peeled copy, as a second one (unmasked) cost 50 more VGPRs and half the occupancy
    if (active) {
      if ((t - t0) & 1) tile(t, R1, std::true_type{}, safe_t);
      else tile(t, R0, std::true_type{}, safe_t);
    }
  };
  pass(std::false_type{});
  // The sum of a query's weights only grows, so a final sum within [lo, hi] bounds every weight
  // and partial sum of the plain pass. bf16: [2^-64, 2^64]; no overflow, and the largest weight is
  // at least 2^-64 / L, far above where bf16 or fp32 lose digits. f16 (largest value 65504,
  // subnormal below 2^-14): [L 2^-12, 2^15]; every weight stays below 65504, and the weights
  // that land among the subnormals (rounding error at most 2^-25 each) move the sum by less than
  // 2^-13 of itself. Any other query (large logits, or NaN) sends its whole block through the
  // safe pass. The last barrier of the pass also frees the ring for the second one.
  constexpr bool half = std::is_same_v<H, f16>;
  const float lo = half ? float(L) * 0x1p-12f : 0x1p-64f, hi = half ? 0x1p15f : 0x1p64f;
  bool redo = false;
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const auto l2 = __builtin_amdgcn_permlane32_swap(__float_as_uint(lsum[qt]), __float_as_uint(lsum[qt]), false, false);
    const float tot = __uint_as_float(l2[0]) + __uint_as_float(l2[1]);
    redo |= active && !(tot >= lo && tot <= hi);
  }
  if (__syncthreads_or(redo)) pass(std::true_type{});

#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const auto l2 = __builtin_amdgcn_permlane32_swap(__float_as_uint(lsum[qt]), __float_as_uint(lsum[qt]), false, false);
    const float tot = __uint_as_float(l2[0]) + __uint_as_float(l2[1]);
    const int qrow = q0 + qt * 32 + l32;
    if (SPLIT && !whole) {
      if (qrow < L) {
        const long row = long(sq) * L + qrow, rows = long(p.seqs) * L;  // dense slice rows
        float* O = p.part + (long(split) * rows + row) * (long(p.heads) * 64) + h * 64;
#pragma unroll
        for (int dt = 0; dt < 2; ++dt)
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4)
            *reinterpret_cast<float4*>(O + dt * 32 + 8 * q4 + 4 * g) =
                make_float4(o[qt][dt][4 * q4], o[qt][dt][4 * q4 + 1], o[qt][dt][4 * q4 + 2], o[qt][dt][4 * q4 + 3]);
        if (g == 0) {
          float* ml = p.part + long(p.nsplit) * rows * p.heads * 64 + ((long(split) * rows + row) * p.heads + h) * 2;
          *reinterpret_cast<float2*>(ml) = make_float2(mref[qt], tot);
        }
      }
      continue;
    }
    const float inv = 1.f / tot;
    if (qrow < L) {
      bf16* O = reinterpret_cast<bf16*>(p.o) + (base + qrow) * p.ldo + h * 64;
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = o[qt][dt][4 * q4 + e] * inv;
          AttnOps<H>::store4(O + dt * 32 + 8 * q4 + 4 * g, v);
        }
    }
  }
}

// ---------------------------------------------------------------------------------------
// fp32 path. 4 waves x 32 queries, 32-key tiles. K and V tiles stream straight into LDS (rows of
// 256 bytes = 64 fp32 head channels, 16-byte chunk c of tile row r in slot c ^ (r & 15)), two
// ring slots each. S^T = K Q^T on v_mfma_f32_32x32x2f32: k-step j pairs head channels j and
// j + 32 (lane half g supplies channel j + 32 g), so a lane reads its key row in 16-byte chunks
// and holds its query's 32 Q values (times log2(e)/8) in registers. The scores' accumulator
// layout (lane l, register r: key 8 (r/4) + 4 g + r%4, query l%32) is the B operand of
// O^T = V^T P^T as it stands: product r takes key 8 (r/4) + 4 g + r%4 in its k-slot g, and the
// A operand reads that key's V row (head channels dt*32 + l%32) with one ds_read_b32. Softmax:
// the max-free plain pass and the running-max safe pass of the bf16 kernel, P in fp32.
template <bool SPLIT>
__global__ void __launch_bounds__(256, 2) attn_f32_kernel(const AttnArgs p, float c) {
  constexpr int TB = 32 * 256;  // one 32-key K or V tile
  __shared__ __attribute__((aligned(1024))) char smem[4 * TB];  // K slots 0, 1 then V slots 0, 1
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, l32 = lane & 31;
  const int L = p.L;
  const int nq = (L + 127) / 128;
  const int ns = SPLIT ? p.nsplit : 1;
  const int id = xcd_contiguous(blockIdx.x, nq * ns * p.heads * p.seqs);
  const int qb = id % nq, split = (id / nq) % ns, h = (id / (nq * ns)) % p.heads, sq = id / (nq * ns * p.heads);
  const long base = long(sq) * p.seq_stride;
  const int q0 = (qb * 4 + wave) * 32;
  const bool active = __builtin_amdgcn_readfirstlane(q0) < L;

  float qf[32];  // Q[query q0 + l32][channels 32 g + (0..31)] * c
  {
    const int qrow = q0 + l32;
    const float* Q = reinterpret_cast<const float*>(p.q) + (base + qrow) * p.ld + h * 64 + 32 * g;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float4 v = qrow < L ? *reinterpret_cast<const float4*>(Q + 4 * i) : make_float4(0.f, 0.f, 0.f, 0.f);
      qf[4 * i] = v.x * c;
      qf[4 * i + 1] = v.y * c;
      qf[4 * i + 2] = v.z * c;
      qf[4 * i + 3] = v.w * c;
    }
  }

  // DMA: load instruction i (0, 1) of wave w fills tile rows 16 i + 4 w + lane/16; lane slot
  // lane%16 holds chunk (lane%16) ^ (row & 15) of that row.
  const float* Kseq = reinterpret_cast<const float*>(p.k) + base * p.ld + h * 64;
  const float* Vseq = reinterpret_cast<const float*>(p.v) + base * p.ld + h * 64;
  const int32x4_t rk = make_rsrc_a(Kseq, uint32_t(long(L) * p.ld * 4));
  const int32x4_t rv = make_rsrc_a(Vseq, uint32_t(long(L) * p.ld * 4));
  int lrw[2];
  uint32_t goff[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    lrw[i] = 16 * i + 4 * wave + (lane >> 4);
    goff[i] = uint32_t(lrw[i] * p.ld * 4 + (((lane & 15) ^ (lrw[i] & 15)) * 16));
  }
  const uint32_t lds0 = uint32_t(reinterpret_cast<uintptr_t>((lds_cptr_a)smem));
  const uint32_t tile_bytes = uint32_t(32 * p.ld * 4);
  auto issue = [&](int t, auto bufc) {
    constexpr int B = decltype(bufc)::value;
    const uint32_t so = uint32_t(t) * tile_bytes;
    const bool full = t * 32 + 32 <= L;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t vo = (full || t * 32 + lrw[i] < L) ? goff[i] : 0x80000000u;
      load_lds_a(rk, vo, so, lds0 + B * TB + (16 * i + 4 * wave) * 256);
      load_lds_a(rv, vo, so, lds0 + (2 + B) * TB + (16 * i + 4 * wave) * 256);
    }
  };

  f32x16 o[2];
  float mref, lsum;
  const int ks = l32 & 15;  // row swizzle of this lane's K row (row l32)

  auto tile = [&](int t, auto bufc, auto masked_t, auto safe_t) {
    constexpr bool masked = decltype(masked_t)::value, safe = decltype(safe_t)::value;
    constexpr int B = decltype(bufc)::value;
    const char* kb = smem + B * TB;
    const char* vb = smem + (2 + B) * TB;
    f32x16 s = {};
    __builtin_amdgcn_s_setprio(1);  // matrix-core sections first among the SIMD's waves (as above)
#pragma unroll
    for (int i = 0; i < 8; ++i) {  // channels 4 i .. 4 i + 3 (+ 32 g)
      const float4 kf = *reinterpret_cast<const float4*>(kb + l32 * 256 + (((8 * g + i) ^ ks) * 16));
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.x, qf[4 * i], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.y, qf[4 * i + 1], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.z, qf[4 * i + 2], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.w, qf[4 * i + 3], s, 0, 0, 0);
    }
    __builtin_amdgcn_s_setprio(0);
    if constexpr (masked) {
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (t * 32 + 8 * (r >> 2) + 4 * g + (r & 3) >= L) s[r] = -INFINITY;
    }
    if constexpr (safe) {
      float mx = s[0];
#pragma unroll
      for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[r]);
      const auto x = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
      mx = fmaxf(__uint_as_float(x[0]), __uint_as_float(x[1]));
      const float mnew = mx > mref + 8.f ? mx : mref;
      if (__builtin_amdgcn_ballot_w64(mnew != mref)) {
        const float alpha = __builtin_amdgcn_exp2f(mref - mnew);
        lsum *= alpha;
#pragma unroll
        for (int r = 0; r < 16; ++r) { o[0][r] *= alpha; o[1][r] *= alpha; }
        mref = mnew;
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = __builtin_amdgcn_exp2f(s[r] - mref);
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = __builtin_amdgcn_exp2f(s[r]);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) lsum += s[r];
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) {
      const int col = dt * 32 + l32;  // head channel of this lane's V reads
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = 8 * (r >> 2) + 4 * g + (r & 3);
        const float vf = *reinterpret_cast<const float*>(vb + key * 256 + (((col >> 2) ^ (key & 15)) * 16) + (col & 3) * 4);
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(vf, s[r], o[dt], 0, 0, 0);
      }
    }
    __builtin_amdgcn_s_setprio(0);
  };

  const int ntiles = (L + 31) / 32;
  const int t0 = SPLIT ? split * p.tps : 0, t1 = SPLIT ? min(ntiles, t0 + p.tps) : ntiles;
  const std::integral_constant<int, 0> R0;
  const std::integral_constant<int, 1> R1;
  auto pass = [&](auto safe_t) {
    mref = decltype(safe_t)::value ? -INFINITY : 0.f;
    lsum = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) { o[0][r] = 0.f; o[1][r] = 0.f; }
    issue(t0, R0);
    wait_vm<0>();
    __syncthreads();
    auto step = [&](int t, auto bufc) {
      constexpr int B = decltype(bufc)::value;
      issue(t + 1, std::integral_constant<int, B ^ 1>{});  // slot B ^ 1 held tile t-1, done by all
      if (active) tile(t, bufc, std::false_type{}, safe_t);
      wait_vm<0>();
      __syncthreads();
    };
    int t = t0;
    for (; t + 2 < t1; t += 2) {
      step(t, R0);
      step(t + 1, R1);
    }
    if (t + 1 < t1) step(t++, R0);
    if (active) {
      if ((t - t0) & 1) tile(t, R1, std::true_type{}, safe_t);
      else tile(t, R0, std::true_type{}, safe_t);
    }
  };
  pass(std::false_type{});
  const auto l0 = __builtin_amdgcn_permlane32_swap(__float_as_uint(lsum), __float_as_uint(lsum), false, false);
  float tot = __uint_as_float(l0[0]) + __uint_as_float(l0[1]);
  if (__syncthreads_or(active && !(tot >= 0x1p-64f && tot <= 0x1p64f))) {
    pass(std::true_type{});
    const auto l1 = __builtin_amdgcn_permlane32_swap(__float_as_uint(lsum), __float_as_uint(lsum), false, false);
    tot = __uint_as_float(l1[0]) + __uint_as_float(l1[1]);
  }

  const int qrow = q0 + l32;
  if (qrow >= L) return;
  if constexpr (SPLIT) {
    const long row = long(sq) * L + qrow, rows = long(p.seqs) * L;  // dense slice rows
    float* O = p.part + (long(split) * rows + row) * (long(p.heads) * 64) + h * 64;
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4)
        *reinterpret_cast<float4*>(O + dt * 32 + 8 * q4 + 4 * g) =
            make_float4(o[dt][4 * q4], o[dt][4 * q4 + 1], o[dt][4 * q4 + 2], o[dt][4 * q4 + 3]);
    if (g == 0) {
      float* ml = p.part + long(p.nsplit) * rows * p.heads * 64 + ((long(split) * rows + row) * p.heads + h) * 2;
      *reinterpret_cast<float2*>(ml) = make_float2(mref, tot);
    }
    return;
  }
  const float inv = 1.f / tot;
  float* O = reinterpret_cast<float*>(p.o) + (base + qrow) * p.ldo + h * 64;
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4)
      *reinterpret_cast<float4*>(O + dt * 32 + 8 * q4 + 4 * g) =
          make_float4(o[dt][4 * q4] * inv, o[dt][4 * q4 + 1] * inv, o[dt][4 * q4 + 2] * inv, o[dt][4 * q4 + 3] * inv);
}

// Merges the key slices of a split launch: per query and head, M = max of the slices' exponent
// references m_s (their maxima, or 0 for a plain pass), O = sum_s 2^(m_s - M) O_s /
// sum_s 2^(m_s - M) l_s. One thread per 8 head channels.
template <typename T>
__global__ void __launch_bounds__(256) attn_combine_kernel(const AttnArgs p) {
  const long rows = long(p.seqs) * p.L;
  const long id = long(blockIdx.x) * 256 + threadIdx.x;
  if (id >= rows * p.heads * 8) return;
  const long row = id / (p.heads * 8);
  const int rem = int(id - row * p.heads * 8), h = rem >> 3, c8 = (rem & 7) * 8;
  if (p.whole > 0) {  // tail split: the whole units wrote their output themselves
    const long sq = row / p.L;
    const int nq = (p.L + p.qrows - 1) / p.qrows;
    if ((sq * p.heads + h) * nq + int(row - sq * p.L) / p.qrows < p.whole) return;
  }
  const long so = rows * p.heads * 64;
  const float* ml = p.part + long(p.nsplit) * so;
  // every slice's loads go out before any is used (one memory latency, not nsplit of them);
  // the sums run in slice order as before
  const int ns = p.nsplit;
  float2 m_l[ATTN_MAX_SPLITS];
  float4 a[ATTN_MAX_SPLITS], b[ATTN_MAX_SPLITS];
#pragma unroll
  for (int s = 0; s < ATTN_MAX_SPLITS; ++s)
    if (s < ns) {
      m_l[s] = *reinterpret_cast<const float2*>(ml + ((s * rows + row) * p.heads + h) * 2);
      const float* src = p.part + s * so + row * p.heads * 64 + h * 64 + c8;
      a[s] = *reinterpret_cast<const float4*>(src);
      b[s] = *reinterpret_cast<const float4*>(src + 4);
    }
  float mx = -INFINITY;
#pragma unroll
  for (int s = 0; s < ATTN_MAX_SPLITS; ++s)
    if (s < ns) mx = fmaxf(mx, m_l[s].x);
  float acc[8] = {}, den = 0.f;
#pragma unroll
  for (int s = 0; s < ATTN_MAX_SPLITS; ++s)
    if (s < ns) {
      const float w = __builtin_amdgcn_exp2f(m_l[s].x - mx);
      den += w * m_l[s].y;
      acc[0] += w * a[s].x; acc[1] += w * a[s].y; acc[2] += w * a[s].z; acc[3] += w * a[s].w;
      acc[4] += w * b[s].x; acc[5] += w * b[s].y; acc[6] += w * b[s].z; acc[7] += w * b[s].w;
    }
  const float inv = 1.f / den;
  const long seq = row / p.L, t = row - seq * p.L;
  T* dst = reinterpret_cast<T*>(p.o) + (seq * p.seq_stride + t) * p.ldo + h * 64 + c8;
#pragma unroll
  for (int k = 0; k < 8; k += 4) {
    const float v[4] = {acc[k] * inv, acc[k + 1] * inv, acc[k + 2] * inv, acc[k + 3] * inv};
    AttnOps<T>::store4(dst + k, v);
  }
}

// Key slices for a long-sequence bf16 launch whose grid would leave the last round of block
// slots mostly empty: S minimises ceil(blocks * S / CUs) / S, the per-CU rounds of 1/S-size
// blocks, plus 2% per slice for the partials and the merge, over S = 1..4 with at least 8 key
// tiles a slice (C4 global 196 -> 172 us with 3 slices, C5 global 2207 -> 2092 us with 3,
// DA3-Small C2 global 122 -> 85 us with 4).
static int attn_splits(long blocks, int ntiles, bool qt2) {
  // Unsplit when the grid is resident at once with at least two blocks a CU (four QT=1 or two
  // QT=2 blocks fit a CU): the merge costs more than the balance it buys (C4 global, 588 blocks:
  // 146 us unsplit against 152 us in 3 slices, measured with the matrix-core wave priorities).
  if (blocks >= 2 * 256 && blocks <= (qt2 ? 2 : 4) * 256) return 1;
  int best = 1;
  double bc = 1e30;
  for (int S = 1; S <= 4; ++S) {
    if (S > 1 && ntiles / S < 8) break;
    const double per_cu = std::ceil(double(blocks) * S / 256.0);
    const double cost = per_cu / S * (1.0 + (S > 1 ? 0.02 * S : 0.0));
    if (cost < bc * 0.999) { bc = cost; best = S; }
  }
  return best;
}

// The launches of a 16-bit (bf16 or f16) attention: the fast kernel, or the generic one for
// strides it does not take; then the slice merge when b is split.
template <typename H>
static void launch16(const Exec& ex, const AttnArgs& b, float c, bool fast, bool qt2, long blocks) {
  const long work = long(b.seqs) * b.L * b.heads * 8;
  const dim3 cgrid(unsigned((work + 255) / 256));
  if (!fast) {
    const dim3 grid(unsigned(cdiv(b.L, ATTN_WAVES * 32) * b.nsplit), b.heads, b.seqs);
    if (b.nsplit > 1) {
      hipLaunchKernelGGL((attn_kernel<H, true>), grid, dim3(ATTN_WAVES * 64), 0, ex.stream, b, c);
      SPLAT_HIP(hipGetLastError());
      hipLaunchKernelGGL(attn_combine_kernel<H>, cgrid, dim3(256), 0, ex.stream, b);
    } else {
      hipLaunchKernelGGL((attn_kernel<H, false>), grid, dim3(ATTN_WAVES * 64), 0, ex.stream, b, c);
    }
    return;
  }
  const dim3 grid(unsigned(b.whole > 0 ? b.whole + (blocks - b.whole) * b.nsplit : blocks * b.nsplit));
  if (b.nsplit > 1) {
    if (qt2) hipLaunchKernelGGL((attn_bf16_kernel<4, 2, true, H>), grid, dim3(256), 0, ex.stream, b, c);
    else hipLaunchKernelGGL((attn_bf16_kernel<4, 1, true, H>), grid, dim3(256), 0, ex.stream, b, c);
    SPLAT_HIP(hipGetLastError());
    hipLaunchKernelGGL(attn_combine_kernel<H>, cgrid, dim3(256), 0, ex.stream, b);
  } else if (qt2) {
    hipLaunchKernelGGL((attn_bf16_kernel<4, 2, false, H>), grid, dim3(256), 0, ex.stream, b, c);
  } else {
    hipLaunchKernelGGL((attn_bf16_kernel<4, 1, false, H>), grid, dim3(256), 0, ex.stream, b, c);
  }
}

void attention(const Exec& ex, const AttnArgs& a) {
  const int ke = a.dt == F32 ? 4 : 8;
  SPLAT_CHECK(a.L > 0 && a.heads > 0 && a.seqs > 0, BAD_ARGUMENT, "attention: bad sizes");
  SPLAT_CHECK(a.ld % ke == 0 && a.ldo % 4 == 0 && a.ld >= (long)a.heads * 64, BAD_ARGUMENT, "attention: strides");
  SPLAT_CHECK(a.seqs == 1 || a.seq_stride >= a.L, BAD_ARGUMENT, "attention: overlapping sequences");
  const bool bf_fast = a.dt != F32 && long(a.L) * a.ld * 2 < 2147483648L && a.ld % 8 == 0 && a.ldo % 4 == 0;
  auto al16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
  const bool f32_fast = a.dt == F32 && long(a.L) * a.ld * 4 < 2147483648L && al16(a.q) && al16(a.k) && al16(a.v) &&
                        al16(a.o);
  // fp32 (and the generic kernels): one block of 128 queries cannot keep a CU busy (fp32
  // matrix cores at 1/16 of the bf16 rate), so a small grid is cut into key slices until it
  // has about two blocks per CU (DA3-Small C1: 66 blocks -> 7 slices).
  const long gblocks = long(cdiv(a.L, ATTN_WAVES * 32)) * a.heads * a.seqs;
  // 4 waves x 32 or 64 queries. Two query sub-tiles per wave (QT = 2) halve the K/V reads per
  // query; four QT=1 or two QT=2 blocks fit a CU. Unsplit launches (L < 4096) take QT = 2 when
  // the most work any CU gets, in QT=1 block units (ceil(blocks / CUs) x QT), is smaller with it,
  // or equal with every CU given a QT=2 block (per shape, with the matrix-core wave priorities:
  // C4 encoder per-view 480 blocks 38.9 vs 40.9 us; C4 info-sharing per-view 360 blocks, C5
  // per-view 1920 and 1440 blocks and C2 per-view 144 blocks all faster on QT=1). Longer
  // sequences: QT = 2 from 500 blocks (C5 global 1.61 vs 1.72 ms; C4 global, 300 such blocks, 156
  // vs 139 us), and when the QT=1 grid has fewer than two blocks a CU and slices anyway (C2 global
  // 66.8 vs 74.6 us).
  const long blocks1 = long(cdiv(a.L, 128)) * a.heads * a.seqs;
  const long blocks2 = long(cdiv(a.L, 256)) * a.heads * a.seqs;
  bool qt2;
  if (a.L >= 4096) {
    qt2 = blocks2 >= 500 || blocks1 < 512;
  } else {
    const long u1 = (blocks1 + 255) / 256, u2 = 2 * ((blocks2 + 255) / 256);
    qt2 = u2 < u1 || (u2 == u1 && blocks2 >= 256);
  }
  const long blocks = qt2 ? blocks2 : blocks1;
  // the fp32 kernel's 32-key tiles: slices of at least 4 tiles, about two blocks per CU
  const int ntiles = f32_fast ? cdiv(a.L, 32) : cdiv(a.L, 64);
  int S = bf_fast    ? (a.L >= 4096 ? attn_splits(blocks, ntiles, qt2) : 1)
                : f32_fast ? int(std::min<long>(std::min<long>(8, std::max(1, ntiles / 4)), std::max<long>(1, cdiv(512, gblocks))))
                           : int(std::min<long>(std::min<long>(8, ntiles / 2), std::max<long>(1, cdiv(512, gblocks))));
  // Tail split: a grid past whole rounds of 256 blocks runs those rounds whole and only the tail
  // in key slices, so that each CU gets about the same work without every block paying for
  // partials and the merge (C4 global, 588 QT=1 blocks: 512 whole, 76 in 3 slices, instead of 76
  // CUs with a third whole block). Modelled like attn_splits and taken when it beats the plan
  // above (unsplit, or every block in S slices) by 3%.
  int whole = 0;
  if (bf_fast && a.L >= 4096 && blocks > 256 && blocks % 256 != 0) {
    const long full = blocks / 256 * 256, tail = blocks - full;
    const double cur = std::ceil(double(blocks) * S / 256.0) / S * (S > 1 ? 1.0 + 0.02 * S : 1.0);
    double best = 1e30;
    int bs = 1;
    for (int s2 = 2; s2 <= 4 && ntiles / s2 >= 8; ++s2) {
      const double cost = std::ceil(double(tail) * s2 / 256.0) / s2 * (1.0 + 0.02 * s2);
      if (cost < best * 0.999) { best = cost; bs = s2; }
    }
    if (bs > 1 && double(full / 256) + best < 0.97 * cur) {
      S = bs;
      whole = int(full);
    }
  }
  AttnArgs b = a;
  if (S > 1) {
    b.tps = cdiv(ntiles, S);
    b.nsplit = cdiv(ntiles, b.tps);  // every slice non-empty
    SPLAT_CHECK(b.nsplit <= ATTN_MAX_SPLITS, BAD_ARGUMENT, "attention: too many key slices");
    const size_t need = size_t(b.nsplit) * a.seqs * a.L * a.heads * (64 + 2) * sizeof(float);
    if (ex.dry && ex.ws) ex.ws->need = std::max(ex.ws->need, need);
    if (!ex.dry && !(ex.ws && ex.ws->ptr && ex.ws->cap >= need)) b.nsplit = 1;  // not sized: one slice
    b.part = b.nsplit > 1 ? static_cast<float*>(ex.ws->ptr) : nullptr;
    if (b.nsplit > 1 && whole > 0) {
      b.whole = whole;
      b.qrows = qt2 ? 256 : 128;  // 4 waves x QT x 32 queries
    }
  }
  if (ex.dry) return;
  const double rows = double(a.seqs) * a.L * a.heads;
  ProfScope ps(ex, "attention", 4.0 * rows * a.L * 64, 4.0 * rows * 64 * (a.dt == F32 ? 4 : 2));
  const float c = a.q_scaled ? 1.f : ATTN_Q_SCALE;  // Q times 1 is exact, rounded or not
  if (f32_fast) {
    const dim3 grid(unsigned(long(cdiv(a.L, 128)) * a.heads * a.seqs * b.nsplit));
    if (b.nsplit > 1) {
      hipLaunchKernelGGL(attn_f32_kernel<true>, grid, dim3(256), 0, ex.stream, b, c);
      SPLAT_HIP(hipGetLastError());
      const long work = long(a.seqs) * a.L * a.heads * 8;
      hipLaunchKernelGGL(attn_combine_kernel<float>, dim3(unsigned((work + 255) / 256)), dim3(256), 0, ex.stream, b);
    } else {
      hipLaunchKernelGGL(attn_f32_kernel<false>, grid, dim3(256), 0, ex.stream, b, c);
    }
  } else if (a.dt == F32) {
    const dim3 grid(unsigned(cdiv(a.L, ATTN_WAVES * 32) * b.nsplit), a.heads, a.seqs);
    if (b.nsplit > 1) {
      hipLaunchKernelGGL((attn_kernel<float, true>), grid, dim3(ATTN_WAVES * 64), 0, ex.stream, b, c);
      SPLAT_HIP(hipGetLastError());
      const long work = long(a.seqs) * a.L * a.heads * 8;
      hipLaunchKernelGGL(attn_combine_kernel<float>, dim3(unsigned((work + 255) / 256)), dim3(256), 0, ex.stream, b);
    } else {
      hipLaunchKernelGGL((attn_kernel<float, false>), grid, dim3(ATTN_WAVES * 64), 0, ex.stream, b, c);
    }
  } else if (a.dt == F16) {
    launch16<f16>(ex, b, c, bf_fast, qt2, blocks);
  } else {
    launch16<bf16>(ex, b, c, bf_fast, qt2, blocks);
  }
  SPLAT_HIP(hipGetLastError());
}

}  // namespace splat
