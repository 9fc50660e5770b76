/* splathip kernel-level entry points: single launches of the hot-path kernels on device
 * buffers, for parity tests and roofline micro-benchmarks. They have no counterpart in the
 * reference (whose kernels are candle's un-vendored matmul and sdpa, called from
 * depthanything3-rs/src/vit_block.rs:49-67 and mapanything-rs/src/vit_block.rs:29-38).
 * All pointers are device pointers; the launch is enqueued on the context's stream. */
#ifndef SPLATHIP_KERNELS_H
#define SPLATHIP_KERNELS_H

#include "splathip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* `dtype` of every entry point below: SPLAT_F32, SPLAT_BF16 or SPLAT_F16 (the storage type of
 * the 16-bit or fp32 operands named as "in `dtype`"); accumulation is fp32 in all three.
 *
 * C[M, N] = act(A[M, K] W[N, K]^T + bias) ; A, W in `dtype`, W with
 * row stride ldw (a multiple of 64, columns K..ldw-1 zero), C fp32 when out_f32 else `dtype`.
 * act: 0 none, 1 relu, 2 gelu (erf). */
int splat_kernel_gemm(splat_ctx* ctx, int dtype, const void* A, int M, int K, const void* W, int N, int ldw,
                      const float* bias, int act, void* C, int out_f32);

/* The pre-norm block's GEMMs with its LayerNorm folded in (depthanything3-rs/src/vit_block.rs:151,165;
 * mapanything-rs/src/vit_block.rs:99,105: norm1 -> qkv, norm2 -> fc1), as the forwards run them.
 * Row statistics: (sum, sum of squares) of each row per group of `group` (64 or 128) columns.
 *  ln_in != NULL (consumer): A [M, K] holds the rows before the norm, ln_in [M, K/group, 2] their
 *    statistics; W and c1 the folded weights (W = gamma (.) W_lin along K, c1[n] = sum_k W[n, k])
 *    and bias = b_lin + W_lin beta; out = act(rstd * (acc - mean * c1[n]) + bias[n]) with each
 *    row's mean and rstd over K (biased variance, eps inside the root); K/group <= 16.
 *  res != NULL (producer, the residual epilogue of proj / fc2): out = res + gamma[n] * (acc +
 *    bias[n]), res and out fp32 [M, N]; with ln_out != NULL also the statistics of the output
 *    rows [M, N/group, 2] and, with copy != NULL, the rows in `dtype` [M, N] (the consumer's A).
 *  Otherwise as splat_kernel_gemm. */
int splat_kernel_gemm_ln(splat_ctx* ctx, int dtype, const void* A, int M, int K, const void* W, int N, int ldw,
                         const float* bias, int act, const float* ln_in, const float* c1, float eps,
                         const float* gamma, const float* res, float* ln_out, void* copy, int group, void* out,
                         int out_f32);

/* Row statistics of fp32 rows x [rows, n] (n a multiple of group, 64 or 128) in the layout above,
 * and the rows converted to `dtype` into copy [rows, n] when copy != NULL. */
int splat_kernel_ln_stats(splat_ctx* ctx, const float* x, int rows, int n, int group, float* stats, int dtype,
                          void* copy);

/* out[s*L + t, h*64 + e] = softmax(q k^T / 8) v for every sequence s < S and head h < heads,
 * reading q, k and v from a [S*L, 3*heads*64] qkv matrix (q | k | v column blocks). In bf16
 * and f16 the kernel multiplies q by log2(e)/8 and rounds it to that type before the products
 * (the networks' qkv GEMMs store q already scaled, rounding once); the weights P go to the
 * matrix cores rounded to the same type. */
int splat_kernel_attention(splat_ctx* ctx, int dtype, const void* qkv, void* out, int S, int L, int heads);

/* splat_kernel_attention that allocates nothing. It has no counterpart in the reference; it is
 * for callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). Same kernels and key-slice plan; the fp32 partials
 * of a key-sliced launch (long sequences) live in a statically allocated scratch of 64 MiB per
 * GPU (ATTN_SCRATCH_BYTES, held by every GPU the library runs on until the process ends)
 * instead of the context's workspace. A launch whose partials would need more than that (e.g.
 * 24889 tokens x 12 heads: 236 MB; 6223 x 12 needs 59 MB and fits) runs as one key slice, with
 * no partials: the same softmax, not bit-identical to the sliced result. Every call on one GPU
 * shares that scratch, which keeps the last call's contents. Eager calls are ordered by the
 * library (each waits, on its stream, for the previous call's kernels on any context of that GPU,
 * through an event; no allocation); calls under stream capture are not, so captured graphs that
 * replay concurrently on one GPU race. Profiling records are not taken. */
int splat_kernel_attention_noalloc(splat_ctx* ctx, int dtype, const void* qkv, void* out, int S, int L, int heads);

/* Convolution (zero padding ks/2) on NHWC maps as an implicit GEMM:
 * out[V, Ho, Wo, Cout] = act(conv(relu_in ? relu(in) : in, w) + bias) + res, with
 * w [Cout, ldw] holding k = (ky*ks + kx)*Cin + ci (candle/PyTorch weight [Cout, Cin, ks, ks]
 * permuted), ldw a multiple of 64 with zero columns past ks*ks*Cin; res NHWC like out or NULL. */
int splat_kernel_conv2d(splat_ctx* ctx, int dtype, const void* in, int V, int H, int W, int Cin, const void* w,
                        int Cout, int ldw, int ks, int stride, const float* bias, int relu_in, int act,
                        const void* res, void* out);

/* Transposed convolution with kernel == stride s on NHWC maps: out[V, R*s, C*s, Cout];
 * w [s*s*Cout, ldw] with row (dy*s + dx)*Cout + co = weight[:, co, dy, dx] (PyTorch weight
 * [Cin, Cout, s, s]); bias [s*s*Cout] (the Cout biases repeated per (dy, dx)). */
int splat_kernel_conv_transpose2d(splat_ctx* ctx, int dtype, const void* in, int V, int R, int C, int Cin,
                                  const void* w, int Cout, int ldw, int s, const float* bias, void* out);

/* Per-kernel-class timing of the following forwards: HIP events around every launch on the
 * context's stream, with each launch's algorithmic work. Graph replay is bypassed while on. */
typedef struct splat_kernel_stat {
  char name[32];
  int launches;
  double ms;     /* summed launch durations */
  double flops;  /* summed algorithmic flops (2 * multiply-adds) */
  double bytes;  /* summed algorithmic bytes (inputs read once + outputs written once) */
} splat_kernel_stat;
int splat_profile_begin(splat_ctx* ctx);
/* Synchronises, stops recording and writes up to `max` classes (largest time first). */
int splat_profile_end(splat_ctx* ctx, splat_kernel_stat* stats, int max, int* count);

/* Bilinear resize with align_corners=True (torch upsample_bilinear2d) of NHWC maps. */
int splat_kernel_resize_bilinear(splat_ctx* ctx, int dtype, const void* in, int V, int Hi, int Wi, int C, void* out,
                                 int Ho, int Wo);

/* The device geometry of splat_da3_reconstruct / splat_ma_reconstruct on given network outputs
 * (all device pointers, fp32 unless noted): DA3 mode when depth != NULL (depth [V,H,W],
 * pose_encoding [V,9]); MapAnything mode otherwise (points_in_camera [V,H,W,3], quaternion
 * [V,4] xyzw, translation [V,3], mask [V,H,W] u8 unambiguous). conf [V,H,W]; foreground
 * [V,H,W] u8 or NULL. Out: cameras [V,16] f64 (R row-major, t, fx, fy, cx, cy, view 0's
 * frame), points [V,H,W,3], conf_out [V,H,W]. */
int splat_kernel_reconstruct(splat_ctx* ctx, int V, int H, int W, const float* depth, const float* pose_encoding,
                             const float* points_in_camera, const float* quaternion, const float* translation,
                             const float* conf, const uint8_t* mask, const uint8_t* foreground, double* cameras,
                             float* points, float* conf_out);

#ifdef __cplusplus
}
#endif

#endif /* SPLATHIP_KERNELS_H */
