/* splathip: MI355X-native (gfx950) feed-forward reconstruction network path of
 * antoineMoPa/splatting-rs (Depth Anything 3 and MapAnything forward), as a C ABI.
 *
 * Each entry point below replaces a reference Rust entry point, named in its comment
 * (file:line under the reference tree). Nothing panics or unwinds across this ABI: every
 * function returns a splat_status and leaves a message for splat_last_error().
 *
 * Threading: a context is not thread-safe; the caller serialises calls on it (the reference's
 * model is used from one thread, depthanything3-rs/src/pipeline.rs:58-73). Contexts are
 * independent; each owns a HIP stream on its device (splat_stream), the loaded weights and an
 * activation arena that grows to the largest input seen. A forward may run independent
 * branches on a second, internal stream of the context; every branch waits for the work
 * enqueued on splat_stream before it and splat_stream waits for the branch before anything
 * enqueued after it, so ordering against splat_stream orders the whole forward.
 *
 * Tensors: images are [V, 3, H, W] float32, ImageNet-normalised, H and W multiples of 14.
 * Host-pointer entry points copy inputs in and outputs out and synchronise before
 * returning. *_device entry points take device pointers (HIP memory on the context's
 * device) and only enqueue on the context's stream (splat_stream); the caller orders the
 * writes of the inputs before the call (e.g. an event on the producing stream waited on by
 * splat_stream, or a device synchronisation), and calls splat_synchronize or synchronises
 * the stream before reading the outputs.
 */
#ifndef SPLATHIP_H
#define SPLATHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct splat_ctx splat_ctx;

typedef enum splat_status {
  SPLAT_OK = 0,
  SPLAT_BAD_ARGUMENT = 1,
  SPLAT_BAD_SHAPE = 2,      /* H or W not a multiple of 14, views of unequal size, ... */
  SPLAT_MISSING_KEY = 3,    /* a checkpoint tensor is absent */
  SPLAT_SHAPE_MISMATCH = 4, /* a checkpoint tensor has the wrong shape */
  SPLAT_HIP_ERROR = 5,
  SPLAT_NONFINITE = 6,      /* output not finite / depth not positive (outputs still written) */
  SPLAT_IO_ERROR = 7,
  SPLAT_NOT_LOADED = 8
} splat_status;

/* The model dtype of the loaders (candle's DType, depthanything3-rs/src/main.rs:60-61,
 * mapanything-rs/src/main.rs:59-60): the storage type of the weights and of the activations the
 * matrix cores read (SPLAT_BF16 and SPLAT_F16 on the 16-bit MFMA instructions, fp32 accumulation;
 * the residual stream stays fp32 in every dtype). */
typedef enum splat_dtype { SPLAT_F32 = 0, SPLAT_BF16 = 1, SPLAT_F16 = 2 } splat_dtype;

/* depthanything3-rs/src/variant.rs:17-23 */
typedef enum splat_da3_variant { SPLAT_DA3_SMALL = 0, SPLAT_DA3_BASE = 1, SPLAT_DA3_LARGE = 2, SPLAT_DA3_GIANT = 3 } splat_da3_variant;

/* depthanything3-rs/src/reference_view.rs:14-22 */
typedef enum splat_ref_strategy { SPLAT_REF_FIRST = 0, SPLAT_REF_MIDDLE = 1, SPLAT_REF_SADDLE_BALANCED = 2 } splat_ref_strategy;

/* depthanything3-rs/src/model.rs:26-34 (Stage::{Block(i), DenseHead, CameraHead}) */
typedef enum splat_stage { SPLAT_STAGE_BLOCK = 0, SPLAT_STAGE_DENSE_HEAD = 1, SPLAT_STAGE_CAMERA_HEAD = 2 } splat_stage;

/* Progress = &mut dyn FnMut(Stage), depthanything3-rs/src/model.rs:34. Called on the calling
 * thread as each stage is enqueued. */
typedef void (*splat_progress_fn)(int stage, int block, void* user);

/* Debug tap: the residual stream [rows, dim] (float32, host memory valid during the call)
 * after backbone / encoder / info-sharing block `block` (blocks numbered across stages).
 * Forces a synchronisation per block. */
typedef void (*splat_tap_fn)(int block, const float* hidden, int rows, int dim, void* user);

/* Debug tap of a block's two residual branches before their LayerScale: branch 0 is the
 * attention branch proj(attn(...)) + bias, branch 1 the feed-forward output fc2(...) + bias
 * (depthanything3-rs/src/vit_block.rs:163-166, mapanything-rs/src/vit_block.rs:103-106), as
 * float32 [rows, dim] host memory valid during the call; rows is the block's own row count
 * (a per-view MapAnything info block leaves out the scale token). Each tap recomputes the
 * branch's last GEMM without the LayerScale and residual epilogue and synchronises. */
typedef void (*splat_branch_tap_fn)(int block, int branch, const float* out, int rows, int dim, void* user);

/* MapAnything widths. The reference hard-codes them (mapanything-rs/src/dinov2.rs:8-17,
 * info_sharing.rs:12-14, dpt.rs:10-14, heads.rs:9-15); ffn: 0 = GELU MLP, 1 = SwiGLU. */
typedef struct splat_ma_spec {
  int enc_dim, enc_heads, enc_depth, enc_ffn, enc_hidden;
  int info_dim, info_heads, info_depth, info_ffn, info_hidden;
  int hooks[3];           /* info blocks whose normed output feeds the dense head; last = depth-1 */
  int dpt_dims[4];        /* 1x1 projection widths per hook */
  int dpt_features;       /* fusion width */
  int pose_dim;           /* pose head width */
  int scale_dim;          /* scale head width */
} splat_ma_spec;

/* Outputs of splat_da3_forward_raw: RawPrediction, depthanything3-rs/src/model.rs:37-49.
 * Caller-owned buffers; NULL skips an optional output. R = H/14, C = W/14. */
typedef struct splat_da3_out {
  float* depth;          /* [V, H, W]  exp(logit)                                         */
  float* depth_conf;     /* [V, H, W]  1 + exp(logit)                                     */
  float* ray_logits;     /* [V, 7, 8R, 8C] (optional)                                     */
  float* pose_encoding;  /* [V, 9] t(3), quaternion xyzw (4), fov (2)                      */
  float* camera_tokens;  /* [V, 2*dim] (optional)                                         */
  int32_t reference_view;/* written by the call                                           */
} splat_da3_out;

/* Outputs of splat_ma_forward: MapAnything::forward's ViewOutput list
 * (mapanything-rs/src/model.rs:21-34, 86-144) plus the raw dense head output. */
typedef struct splat_ma_out {
  float* raw;            /* [V, 6, H, W] dense head output before activation (optional)   */
  float* quaternion;     /* [V, 4] unit (x, y, z, w), camera to world                      */
  float* translation;    /* [V, 3] metric (times the scale)                                */
  float* scale;          /* [1] metric scale                                               */
  float* points;         /* [V, H, W, 3] camera-frame points (optional)                    */
  float* conf;           /* [V, H, W] 1 + exp(raw conf) (optional)                         */
  uint8_t* mask;         /* [V, H, W] unambiguous (raw mask logit > 0) (optional)          */
} splat_ma_out;

/* Outputs of the post-forward reconstructions: one point map and camera per view, all in view
 * 0's camera frame (OpenCV axes), as depthanything3-rs/src/pipeline.rs:17-42 (Camera,
 * ReconstructedView) and mapanything-rs/src/reconstruction.rs:8-19. Caller-owned host
 * buffers; NULL skips an optional field. */
typedef struct splat_recon_out {
  float* points;            /* [V, H, W, 3] scene points (required)                          */
  float* conf;              /* [V, H, W] confidence after multi-view cleaning (required)     */
  float* depth;             /* [V, H, W] camera-frame depth (optional)                       */
  double* rotation;         /* [V, 3, 3] camera to scene, row-major (optional)               */
  double* translation;      /* [V, 3] (optional)                                             */
  double* focal;            /* [V, 2] fx, fy in pixels (optional)                            */
  double* principal_point;  /* [V, 2] cx, cy (optional)                                      */
  int32_t reference_view;   /* DA3: the network's reference view; MapAnything: 0             */
} splat_recon_out;

/* --- context ------------------------------------------------------------------------------ */

/* Replaces candle's `Device::new_metal(0)` / `Device::Cpu` choice (depthanything3-rs/src/main.rs:136). */
int splat_create(int hip_device, splat_ctx** out);
void splat_destroy(splat_ctx* ctx);
/* Last error message of the context ("" when none). With ctx == NULL: of the last failed splat_create. */
const char* splat_last_error(const splat_ctx* ctx);
/* The context's hipStream_t, for event timing and device-pointer entry points. */
void* splat_stream(splat_ctx* ctx);
int splat_synchronize(splat_ctx* ctx);
/* 1 = capture each forward shape into a HIP graph on first use and replay it (default 0).
 * Ignored while progress callbacks, debug taps or branch taps are set. */
int splat_set_graphs(splat_ctx* ctx, int enable);
/* Per-block residual taps (NULL to disable); replaces nothing in the reference: a test hook. */
int splat_set_debug_taps(splat_ctx* ctx, splat_tap_fn fn, void* user);
/* Per-block branch taps (NULL to disable), a test hook like splat_set_debug_taps: the reference
 * has no counterpart; they make a block's arithmetic visible where LayerScale 1e-5 leaves the
 * residual stream nearly unchanged. */
int splat_set_branch_taps(splat_ctx* ctx, splat_branch_tap_fn fn, void* user);

/* mapanything-rs/src/image_input.rs:195-216 (to_model_input, used by both crates' preprocess):
 * host RGBA u8 [V, H, W, 4] (already resized and cropped) -> device images [V, 3, H, W] f32,
 * ImageNet-normalised, and device foreground [V, H, W] u8 = alpha >= 128 (NULL: skipped).
 * Uploads 4 bytes per pixel instead of 12. A view without a pixel of alpha >= 128 is the
 * reference's error (image_input.rs:197 "fully transparent after cropping"): SPLAT_BAD_ARGUMENT
 * naming the view, as for the two model_inputs entry points below. Synchronises splat_stream. */
int splat_to_model_input(splat_ctx* ctx, const uint8_t* rgba, int V, int H, int W, float* images, uint8_t* foreground);

/* --- image preprocessing: the crates' load_images from decoded RGBA onwards, on the device ---- */

/* image 0.25.10 imageops::FilterType values the crates resize with (Cargo.lock:2536-2539). */
enum { SPLAT_FILTER_TRIANGLE = 1, SPLAT_FILTER_CATMULLROM = 2, SPLAT_FILTER_LANCZOS3 = 3 };

/* image::imageops::resize as DynamicImage::resize_exact runs it on an RGBA8 image (called at
 * depthanything3-rs/src/preprocess.rs:56 and mapanything-rs/src/preprocess.rs:52-56): host RGBA8
 * [height, width, 4] -> host RGBA8 [new_height, new_width, 4], computed on the device (separable
 * rows-then-columns passes with the crate's f32 weights, rounded and clamped to u8; a copy at
 * the same size). */
int splat_resize_rgba8(splat_ctx* ctx, const uint8_t* src, int width, int height, uint8_t* dst, int new_width,
                       int new_height, int filter);
/* depthanything3-rs/src/preprocess.rs:36-45 model_input_size: the longest side to 504, then each
 * side to the nearest multiple of 14 (no context needed; errors in splat_last_error(NULL)). */
int splat_da3_input_size(int width, int height, int* bounded_width, int* bounded_height, int* out_width,
                         int* out_height);
/* mapanything-rs/src/preprocess.rs:31-41 input_size: the size of the table entry closest to the
 * mean aspect ratio of n images. */
int splat_ma_input_size(int n, const int* widths, const int* heights, int* out_width, int* out_height);
/* depthanything3-rs/src/preprocess.rs:86-123 model_inputs_from_cutouts from the decoded images on:
 * each host RGBA8 image k [heights[k], widths[k], 4] resized as resize_for_model (to the bounded
 * size, then to the patch multiples; CatmullRom to enlarge, Triangle to shrink), all center
 * cropped to the smallest size among them, then to_model_input: device images [n, 3, H, W] f32
 * ImageNet-normalised and device foreground [n, H, W] u8 (NULL: skipped). images must hold n*3*H*W
 * floats for the (H, W) that splat_da3_input_size and the minimum over the images give; *out_height
 * and *out_width receive it. */
int splat_da3_model_inputs(splat_ctx* ctx, int n, const uint8_t* const* rgba, const int* widths, const int* heights,
                           float* images, uint8_t* foreground, int* out_height, int* out_width);
/* mapanything-rs/src/preprocess.rs:66-80 load_images from the decoded images on: every image
 * resized to cover splat_ma_input_size's (W, H) (Lanczos3 to shrink, CatmullRom to enlarge) and
 * center cropped to it (cover_and_crop, :43-63), then to_model_input, as splat_da3_model_inputs. */
int splat_ma_model_inputs(splat_ctx* ctx, int n, const uint8_t* const* rgba, const int* widths, const int* heights,
                          float* images, uint8_t* foreground, int* out_height, int* out_width);

/* --- Depth Anything 3 ------------------------------------------------------------------------ */

/* weights::load_model(variant, strategy, Some(path), dtype, device), depthanything3-rs/src/weights.rs:26-48
 * (tensors under the `model.` prefix, every shape checked as DepthAnything3::new does,
 * depthanything3-rs/src/model.rs:85-94). */
int splat_load_da3(splat_ctx* ctx, const char* safetensors_path, int variant, int dtype, int ref_strategy);
/* weights::model_from_safetensors_bytes, depthanything3-rs/src/weights.rs:51-60 (bytes are copied). */
int splat_load_da3_bytes(splat_ctx* ctx, const uint8_t* bytes, size_t len, int variant, int dtype, int ref_strategy);
/* DepthAnything3::forward_raw_with_progress, depthanything3-rs/src/model.rs:101-123 (progress may be NULL). */
int splat_da3_forward_raw(splat_ctx* ctx, const float* images, int V, int H, int W, splat_progress_fn progress,
                          void* user, splat_da3_out* out);
/* Same with device pointers in `images` and in every non-NULL field of `out` except
 * reference_view, which is written to *ref_view_device (int32 device memory) when not NULL. */
int splat_da3_forward_raw_device(splat_ctx* ctx, const float* images, int V, int H, int W, splat_da3_out* out,
                                 int32_t* ref_view_device);

/* depthanything3-rs/src/pipeline.rs:52-133 (reconstruct): forward, per-view camera from the pose
 * encoding, poses relative to view 0, depth unprojected through each view's intrinsics, then
 * mapanything-rs/src/cleaning.rs:28-64 (zero the confidence of points in front of another
 * view's more confident foreground). Geometry runs on the device. foreground: [V, H, W]
 * (non-zero = foreground; NULL = every pixel, the reference's opaque images). Returns
 * SPLAT_NONFINITE (outputs written) where DepthAnything3::forward asserts (model.rs:139-146). */
int splat_da3_reconstruct(splat_ctx* ctx, const float* images, int V, int H, int W, const uint8_t* foreground,
                          splat_recon_out* out);

/* --- MapAnything ----------------------------------------------------------------------------- */

/* MapAnything::new(VarBuilder over the checkpoint), mapanything-rs/src/model.rs:69-81;
 * spec NULL = the reference's constants. */
int splat_load_mapanything(splat_ctx* ctx, const char* safetensors_path, const splat_ma_spec* spec, int dtype);
int splat_load_mapanything_bytes(splat_ctx* ctx, const uint8_t* bytes, size_t len, const splat_ma_spec* spec, int dtype);
/* The reference's constants (spec NULL above). */
void splat_ma_reference_spec(splat_ma_spec* out);
/* MapAnything::forward(images, intrinsics), mapanything-rs/src/model.rs:86-144, for views of
 * one size. intrinsics: NULL (every camera unknown) or host [V, 4] doubles fx, fy, cx, cy
 * (pixels, pixel centres at integer coordinates) per view; a view whose fx or fy is not a
 * finite positive number is unknown (Option::None in the reference). Known views add the ray
 * encoder's features (ray_encoder.rs:78-86, fp32) to their patches (model.rs:97-102);
 * SPLAT_MISSING_KEY if the checkpoint has no ray_dirs_encoder. */
int splat_ma_forward(splat_ctx* ctx, const float* images, int V, int H, int W, const double* intrinsics,
                     splat_ma_out* out);
/* Same with device pointers in `images` and `out`; `intrinsics` stays a host array. */
int splat_ma_forward_device(splat_ctx* ctx, const float* images, int V, int H, int W, const double* intrinsics,
                            splat_ma_out* out);
/* mapanything-rs/src/pipeline.rs:41-104 (reconstruct): forward (intrinsics as splat_ma_forward),
 * poses relative to view 0, fit_intrinsics on the camera-frame points (pipeline.rs:18-39),
 * ambiguous pixels' confidence zeroed, then the multi-view cleaning; focal = (fx, fy) of the
 * fit (the reference's Camera keeps their mean). Geometry runs on the device. */
int splat_ma_reconstruct(splat_ctx* ctx, const float* images, int V, int H, int W, const double* intrinsics,
                         const uint8_t* foreground, splat_recon_out* out);
/* Dinov2::forward for every view (mapanything-rs/src/dinov2.rs:129-145): tokens [V, 1+R*C, enc_dim]. */
int splat_ma_encode(splat_ctx* ctx, const float* images, int V, int H, int W, float* tokens);
int splat_ma_encode_device(splat_ctx* ctx, const float* images, int V, int H, int W, float* tokens);

#ifdef __cplusplus
}
#endif

#endif /* SPLATHIP_H */
