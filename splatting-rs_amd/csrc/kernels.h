// Host-side launchers of the splathip HIP kernels. All tensors are device pointers; all
// activations are row-major token matrices [rows, channels] or NHWC feature maps
// [views, rows, cols, channels] (a token matrix of a patch grid IS its NHWC map).
#pragma once

#include <functional>
#include "common.h"

namespace splat {

enum Dtype { F32 = 0, BF16 = 1, F16 = 2 };  // the C API's splat_dtype values
inline size_t dtype_size(int dt) { return dt == F32 ? 4 : 2; }

enum Act { ACT_NONE = 0, ACT_RELU = 1, ACT_GELU = 2 };
enum AMode { A_ROWS = 0, A_CONV = 1 };
enum StoreMode { STORE_ROWS = 0, STORE_CONVT = 1 };

// C[m, n] = epilogue(sum_k A[m, k] * W[n, k]).
//
// A (dtype `dt`): A_ROWS -> row-major [M, lda]; A_CONV -> implicit im2col of an NHWC map
// [V, Hi, Wi, Cin] for a ks x ks convolution (stride, pad), k = (ky*ks + kx)*Cin + ci.
// W (dtype `dt`): [N, ldw] row-major; columns K..ldw-1 must be zero and ldw a multiple of 64.
// Epilogue, in this order: folded LayerNorm (ln_in, below); + bias[n]; activation; + addtab[(m % period) * N + n];
// * gamma[n]; + res[row, n]; + res2[row, n]; store (`out_f32` selects fp32 or `dt`).
// With rm_P > 0 the stored row is (m / rm_P) * rm_n + rm_off + m % rm_P (also for res/res2).
// STORE_CONVT scatters a kernel=stride transposed convolution: m = (v, r, c) of an R x C
// input grid, n = (dy*s + dx)*Cout + co -> out NHWC [V, R*s, C*s, Cout].
struct GemmArgs {
  int dt = BF16;
  int M = 0, N = 0, K = 0;
  const void* A = nullptr; long lda = 0;
  int amode = A_ROWS;
  int V = 0, Hi = 0, Wi = 0, Cin = 0, Ho = 0, Wo = 0, ks = 3, stride = 1, pad = 1;
  int relu_in = 0;
  const void* W = nullptr; long ldw = 0;
  const float* bias = nullptr;
  int act = ACT_NONE;
  const float* addtab = nullptr; int addtab_period = 1;
  const float* gamma = nullptr;
  const void* res = nullptr; long ldres = 0; int res_f32 = 0;
  const void* res2 = nullptr; long ldres2 = 0; int res2_f32 = 0;
  int act_post = ACT_NONE;  // activation applied after the residual adds
  void* out = nullptr; long ldc = 0; int out_f32 = 0;
  int rm_P = 0, rm_n = 0, rm_off = 0;
  int store = STORE_ROWS;
  int ct_s = 1, ct_R = 0, ct_C = 0, ct_Cout = 0;
  int epi_vec = 0;  // set by gemm(): the epilogue may use 16-byte vector accesses
  // Set by the launcher: tiles are walked in groups of tgroup tile rows (column by column inside
  // a group); with tcontig each XCD takes a contiguous run of that order, else the round-robin deal.
  int tgroup = 8, tcontig = 0;
  // Set by gemm() for a split-K launch: fp32 partial sums [splits][M][ldp], kper k-tiles each.
  float* part = nullptr; long ldp = 0; int kper = 0;
  // MapAnything output head fused into the epilogue (bf16 convolution with N = 128, act ReLU):
  // h = relu(acc + bias) rounded to bf16 as a stored map would be, raw = hw3 [6, 128] h + hb3,
  // then what pointwise_head(PW_MA) writes from raw: ho0 raw NCHW [V, 6, hhw], ho1 points
  // [pix, 3] (scaled by *hscale), ho2 confidence, ho3 unambiguous mask (each may be null).
  const float* hw3 = nullptr; const float* hb3 = nullptr; const float* hscale = nullptr; int hhw = 0;
  float* ho0 = nullptr; float* ho1 = nullptr; float* ho2 = nullptr; uint8_t* ho3 = nullptr;
  // Pre-norm LayerNorm folded into the GEMMs on either side of it (a block's LN -> linear).
  // Producer (ln_out != null; N a multiple of ln_group, 64 or 128): also writes the statistics
  //   of its final output rows, ln_out[(m * (N / ln_group) + g) * 2 + {0, 1}] = (sum, sum of
  //   squares) of row m over columns [g * ln_group, (g + 1) * ln_group), and when ln_copy !=
  //   null the output rows in the GEMM's dtype, [M, ldc] (the consumer's A operand in bf16).
  // Consumer (ln_in != null): A holds the rows x before the norm (K columns); row m's mean and
  //   rstd come from its ln_parts (<= 16) partials in ln_in (biased variance over K, eps
  //   ln_eps) and the epilogue starts from rstd * (acc - mean * ln_c1[n]) + bias[n].
  //   W = gamma (.) W_linear (scaled along K), ln_c1[n] = sum_k W[n, k], bias = b_linear +
  //   W_linear beta, folded at load: linear(LN(x)) up to rounding. Needs plain rows (no
  //   residual, remap or table) and runs without split-K.
  float* ln_out = nullptr; int ln_group = 64; void* ln_copy = nullptr;
  const float* ln_in = nullptr; int ln_parts = 0; const float* ln_c1 = nullptr; float ln_eps = 0.f;
  // qk-norm + 2D RoPE of a DA3 qkv GEMM (depthanything3-rs/src/vit_block.rs:155-162,
  // rope.rs:57-73), applied to the q and k columns in the epilogue (qk_dim = d > 0, N = 3 d,
  // heads of 64 columns, needs a folded-LayerNorm consumer): per head LayerNorm over its 64
  // channels (eps 1e-5; qw/qb, kw/kb [64], null: no norm), then with rope_cs != null the
  // rotation of channel pairs (c, c + 16) within each 32-channel half, channels 0-31 by the
  // token's row position and 32-63 by its column position; rope_cs [npos][16] cos then
  // [npos][16] sin. Token t = m % rope_n: t = 0 at (0, 0), patch t at ((t-1) / rope_cols + 1,
  // (t-1) % rope_cols + 1), or (1, 1) with rope_across.
  // SwiGLU gate of a w12 GEMM (mapanything-rs/src/vit_block.rs:64-70) in the epilogue (needs a
  // folded-LayerNorm consumer): W rows (and bias) interleaved in chunks of 8, x1 rows 8j..8j+7
  // then the matching x2 rows (Loader::linear_ln), N = 2 * hidden; out [M, ldc] holds
  // silu(x1) * x2, hidden columns.
  int glu = 0;
  int qk_dim = 0; const float* qw = nullptr; const float* qb = nullptr; const float* kw = nullptr;
  const float* kb = nullptr; const float* rope_cs = nullptr; int rope_n = 1, rope_cols = 1, rope_across = 0,
  rope_npos = 0;
  // Output columns [0, q_cols) times q_scale, last before the store (after the qk-norm and
  // RoPE; needs a folded-LayerNorm consumer, q_cols a multiple of 8): a qkv GEMM hands the
  // attention Q already multiplied by its softmax scale (AttnArgs::q_scaled).
  int q_cols = 0; float q_scale = 1.f;
};
// A producer whose tile path cannot emit the statistics (split-K, unaligned, tiles narrower
// than the group) gets them (and the copy) from ln_stats() on its output.
void gemm(const Exec& ex, const GemmArgs& a);

// Row statistics of fp32 rows in the layout of GemmArgs::ln_out ((sum, sum of squares) per
// group of `group` columns, 64 or 128; n a multiple of it) and, when copy != null, the rows
// converted to copy_dt (same row stride). Row r of the launch is row (r / rm_P) * rm_n +
// rm_off + r % rm_P (rm_P > 0) or r, for the input, the statistics and the copy alike.
void ln_stats(const Exec& ex, const float* x, long ldx, int rows, int n, int group, float* stats, int copy_dt,
              void* copy, int rm_P = 0, int rm_n = 0, int rm_off = 0);

// Flash attention, head dim 64, no mask: O = softmax(Q K^T / 8) V per (sequence, head).
// Row t of sequence s is row s*seq_stride + t of q/k/v (row stride ld elements, head h at
// column h*64); O rows likewise with stride ldo.
struct AttnArgs {
  int dt = BF16;
  const void* q = nullptr; const void* k = nullptr; const void* v = nullptr; long ld = 0;
  void* o = nullptr; long ldo = 0;
  int L = 0, heads = 0, seqs = 1; long seq_stride = 0;
  // Set by attention() for a key-split launch: nsplit slices of tps 64-key tiles each; part
  // holds the unnormalised fp32 O of every slice, [nsplit][seqs*L][heads*64], then each
  // slice's (exponent reference, sum) per query and head, [nsplit][seqs*L][heads][2].
  int nsplit = 1, tps = 0; float* part = nullptr;
  // Tail split (a bf16/f16 launch with nsplit > 1): the first `whole` (query block, head,
  // sequence) units, query blocks of qrows queries fastest, run over every key tile and write O
  // themselves; only the remaining units run in slices (and go through part).
  int whole = 0, qrows = 0;
  // Q already multiplied by log2(e)/8 (ATTN_Q_SCALE) and rounded once; otherwise the bf16
  // kernel multiplies each Q element by it and rounds it to bf16 again (a second rounding).
  int q_scaled = 0;
};
constexpr float ATTN_Q_SCALE = 0.125f * 1.4426950408889634f;
void attention(const Exec& ex, const AttnArgs& a);

// Statically allocated device scratch for the key-slice partials of attention launches that
// may not allocate: ATTN_SCRATCH_BYTES on every GPU the library runs on. attention_scratch()
// returns its address on `device` (looked up on first use, which must be with that device
// current); an Exec whose ws points at {that address, ATTN_SCRATCH_BYTES} runs attention()
// on it.
constexpr size_t ATTN_SCRATCH_BYTES = size_t(64) << 20;
constexpr int ATTN_SCRATCH_DEVICES = 64;
void* attention_scratch(int device);
// Runs `launch` (kernels on `stream` that use the device's scratch) after the previous eager
// launch that used it, on whatever stream or context that ran, and leaves an event behind for the
// next: calls from several contexts on one GPU are ordered by their host order. A launch under
// stream capture is left to the caller's graph to order. Allocates nothing.
void attention_scratch_ordered(int device, hipStream_t stream, const std::function<void()>& launch);

// LayerNorm over the last dim of rows: out[r] = LN(in[row_in(r)]) * w + b (w/b nullable);
// row_in(r) = (r / rm_P) * rm_n + rm_off + r % rm_P when rm_P > 0, else r.
void layer_norm(const Exec& ex, int in_dt, const void* in, long ldin, int out_dt, void* out, long ldout,
                int rows, int n, const float* w, const float* b, float eps, int rm_P = 0, int rm_n = 0,
                int rm_off = 0);

// images fp32 [V,3,H,W] -> patch matrix [V*R*C, kpad] (dtype dt), k = c*196 + ky*14 + kx.
void im2col_patch(const Exec& ex, int dt, const float* img, int V, int H, int W, void* out, int kpad);

// xs[v*n + 0, :] = cls[:] + pos0[:] (fp32) for every view v.
void write_class_rows(const Exec& ex, float* xs, int V, int n, int dim, const float* cls, const float* pos0);

// Bilinear, align_corners=True, NHWC: sample grid computed for (Hf, Wf) outputs, the first
// (Ho, Wo) of them written (crop). Optional + addtab[(oy*Wo+ox)*C + c] and relu.
void resize_bilinear(const Exec& ex, int dt, const void* in, int V, int Hi, int Wi, int C, void* out, int Hf,
                     int Wf, int Ho, int Wo, const float* addtab, int relu);

// Pointwise output heads on an NHWC map [pix = V*H*W, Cin] (dt):
//  PW_DEPTH: l = W x + b (2 ch) -> o0[pix] = exp(l0), o1[pix] = 1 + exp(l1)         (fp32)
//  PW_RAY  : x' = relu(LN(x) no affine, eps 1e-5); o0 NCHW [V, Cout, H*W] = W x' + b   (fp32)
//  PW_MA   : raw = W x + b (6 ch) -> o0 NCHW raw [V,6,H*W]; with scale (device scalar):
//            points o1 [pix,3], conf o2 [pix], mask o3 (uint8) [pix]
enum PwMode { PW_DEPTH = 0, PW_RAY = 1, PW_MA = 2 };
void pointwise_head(const Exec& ex, int dt, int mode, const void* in, long pix, int hw, int cin, int cout,
                    const float* w, const float* b, float* o0, float* o1, float* o2, uint8_t* o3,
                    const float* scale);

// y[m, n] = act(sum_k x[m*ldx + k] * W[n, k] + b[n]) for a handful of rows; x, y fp32,
// W dtype wdt ([N, ldw]).
void small_linear(const Exec& ex, int wdt, const float* x, long ldx, int M, int K, const void* W, long ldw,
                  const float* b, float* y, long ldy, int N, int act);

// DA3 reference-view choice on the device (saddle-balanced / first / middle) from the class
// tokens xs[v*n, :dim] (fp32); writes the index to *ref.
void select_reference_view(const Exec& ex, const float* xs, int V, int n, int dim, int strategy, int* ref);
// xs[v*n] = cam[ref == v ? 0 : 1] (cam: [2, dim] fp32).
void set_camera_tokens(const Exec& ex, float* xs, int V, int n, int dim, const float* cam, const int* ref);

// DA3 hook: for every view and patch token t (1..n-1):
//   h = cat(within[t], LN_{bn}(xs[t])) (2*dim), out[v*P + t-1] = LN_{hn}(h)  (dtype dt)
// and when cam_out != null: cam_out[v] = cat(within[v*n], xs[v*n]) (fp32, no norm).
void da3_hook(const Exec& ex, int dt, const float* within, const float* xs, int V, int n, int dim,
              const float* bnw, const float* bnb, const float* hnw, const float* hnb, void* out, float* cam_out);

// Known-camera rays (mapanything-rs/src/model.rs:38-54) already pixel-unshuffled by 14
// (ray_encoder.rs:48-54): out [V, H/14, W/14, 588] fp32, channel c*196 + 14*i + j for ray
// component c of pixel (14*row + i, 14*col + j). cam [V, 5] f64 device: fx, fy, cx, cy, known.
void ray_unshuffled(const Exec& ex, const double* cam, int V, int H, int W, float* out);
// xs[v*n + 1 + p, :] += feat[v*P + p, :] for the views whose cam[v, 4] != 0.
void add_view_features(const Exec& ex, float* xs, int V, int n, int P, int dim, const float* feat, const double* cam);

// Post-forward geometry, all on the device (depthanything3-rs/src/pipeline.rs:44-133,
// mapanything-rs/src/pipeline.rs:18-104, cleaning.rs:28-64). DA3: depth [V,H,W] and
// pose_enc [V,9]; MapAnything (depth NULL): camera-frame points pts_cam [V,H,W,3], xyzw quat
// [V,4], metric trans [V,3], unambiguous mask, fitted [V,4] scratch. conf [V,H,W] in;
// fg [V,H,W] foreground (NULL = all). Out: cam [V,16] (R row-major, t, fx, fy, cx, cy in
// view 0's frame), conf0 scratch, points [V,H,W,3] in view 0's frame, cleaned conf_out.
void reconstruct_geometry(const Exec& ex, int V, int H, int W, const float* depth, const float* pose_enc,
                          const float* pts_cam, const float* quat, const float* trans, const float* conf,
                          const uint8_t* mask, const uint8_t* fg, double* cam, double* fitted, float* conf0,
                          float* points, float* conf_out);

// RGBA u8 [V,H,W,4] -> normalised images [V,3,H,W] f32 and foreground [V,H,W] (NULL: skipped).
void to_model_input(const Exec& ex, const uint8_t* rgba, int V, int H, int W, float* img, uint8_t* fg);
// flags[v] = 1 if view v of the RGBA8 batch has a pixel with alpha >= 128, else 0.
void foreground_any(const Exec& ex, const uint8_t* rgba, int V, int H, int W, int* flags);

// The taps of one resize axis on the device: output coordinate o reads count[o] inputs from
// first[o], weights w[offset[o] .. offset[o] + count[o]) (normalised, f32).
struct ResizeTaps {
  const int* first = nullptr; const int* count = nullptr; const int* offset = nullptr; const float* w = nullptr;
};
// RGBA8 [H, W, 4] -> RGBA8 [NH, NW, 4] by image 0.25.10's separable resize: rows (vertical
// taps, f32 tmp [NH, W, 4]) then columns (horizontal taps, rounded and clamped to u8).
void resize_rgba8(const Exec& ex, const uint8_t* src, int W, int H, float* tmp, uint8_t* dst, int NW, int NH,
                  const ResizeTaps& rows, const ResizeTaps& cols);

// Generic elementwise helpers.
void convert(const Exec& ex, int in_dt, const void* in, int out_dt, void* out, long count);
// Row r, column c of in (row stride ldi elements) -> out (row stride ldo), converted.
void convert_rows(const Exec& ex, int in_dt, const void* in, long ldi, int out_dt, void* out, long ldo, int rows,
                  int cols);
void add_rows(const Exec& ex, float* xs, int rows, int dim, const float* vec);           // xs[r] += vec
void copy_rows_f32(const Exec& ex, float* dst, long lddst, const float* src, long ldsrc, int rows, int dim);
// mean over groups of P rows: out[g, c] = mean_p in[g*P + p, c] (fp32 out)
void mean_rows(const Exec& ex, int dt, const void* in, int groups, int P, int C, float* out);
// MA scale head tail + pose quaternion normalisation happen in small kernels:
void exp_clamp(const Exec& ex, float* x, int count, float lo);
void normalize_rows(const Exec& ex, float* x, int rows, int dim, float min_norm);
void scale_rows(const Exec& ex, const float* x, int rows, int dim, const float* scale, float* out);

}  // namespace splat
