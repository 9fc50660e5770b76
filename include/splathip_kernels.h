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

/* C[M, N] = act(A[M, K] W[N, K]^T + bias) ; A, W in `dtype` (SPLAT_F32 / SPLAT_BF16), W with
 * row stride ldw (a multiple of 64, columns K..ldw-1 zero), C fp32 when out_f32 else `dtype`.
 * act: 0 none, 1 relu, 2 gelu (erf). */
int splat_kernel_gemm(splat_ctx* ctx, int dtype, const void* A, int M, int K, const void* W, int N, int ldw,
                      const float* bias, int act, void* C, int out_f32);

/* out[s*L + t, h*64 + e] = softmax(q k^T / 8) v for every sequence s < S and head h < heads,
 * reading q, k and v from a [S*L, 3*heads*64] qkv matrix (q | k | v column blocks). */
int splat_kernel_attention(splat_ctx* ctx, int dtype, const void* qkv, void* out, int S, int L, int heads);

#ifdef __cplusplus
}
#endif

#endif /* SPLATHIP_KERNELS_H */
