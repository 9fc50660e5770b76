// The C ABI (include/splathip.h): argument checks, error mapping and host<->device staging
// around the models. Nothing throws across this boundary.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>

#include "runtime.h"
#include "../../include/splathip_kernels.h"

using namespace splat;

namespace {

thread_local std::string g_create_error;

Context* C(splat_ctx* c) { return reinterpret_cast<Context*>(c); }

// Entry points without a context: errors go where splat_last_error(NULL) reads them.
template <typename F>
int guard_free(F&& fn) {
  try {
    fn();
    return OK;
  } catch (const Error& e) {
    g_create_error = e.what();
    return e.code;
  } catch (const std::exception& e) {
    g_create_error = e.what();
    return HIP_ERROR;
  }
}

template <typename F>
int guard(Context* ctx, F&& fn) {
  if (!ctx) return BAD_ARGUMENT;
  try {
    SPLAT_HIP(hipSetDevice(ctx->device));
    fn();
    ctx->last_error.clear();
    return OK;
  } catch (const Error& e) {
    ctx->last_error = e.what();
    return e.code;
  } catch (const std::exception& e) {
    ctx->last_error = e.what();
    return HIP_ERROR;
  } catch (...) {
    ctx->last_error = "unknown error";
    return HIP_ERROR;
  }
}

// splat_dtype -> the library's storage type (the values agree; unknown values are rejected)
int model_dtype(int dtype) {
  SPLAT_CHECK(dtype == SPLAT_F32 || dtype == SPLAT_BF16 || dtype == SPLAT_F16, BAD_ARGUMENT, "unknown dtype");
  return dtype == SPLAT_F32 ? F32 : dtype == SPLAT_F16 ? F16 : BF16;
}

void check_images(const float* images, int V, int H, int W) {
  SPLAT_CHECK(images != nullptr, BAD_ARGUMENT, "images is NULL");
  SPLAT_CHECK(V >= 1, BAD_SHAPE, "no views");
  SPLAT_CHECK(H >= 14 && W >= 14 && H % 14 == 0 && W % 14 == 0, BAD_SHAPE,
              "image " + std::to_string(W) + "x" + std::to_string(H) + " is not a multiple of the 14 px patch");
}

void* staging(Context* ctx, int slot, size_t bytes) { return ctx->staging_buffer(slot, bytes); }

bool use_graphs(Context* ctx) { return ctx->graphs && !ctx->hooks.any() && !ctx->ex.prof; }

void da3_device(Context* ctx, const float* images, int V, int H, int W, const splat_da3_out& out, int32_t* ref) {
  SPLAT_CHECK(ctx->da3 != nullptr, NOT_LOADED, "no Depth Anything 3 model loaded");
  check_images(images, V, H, W);
  SPLAT_CHECK(out.depth && out.depth_conf && out.pose_encoding, BAD_ARGUMENT, "depth, depth_conf and pose_encoding are required");
  ctx->da3->prepare(V, H, W);
  Context::GraphKey key{0, V, H, W, images, {out.depth, out.depth_conf, out.ray_logits, out.pose_encoding, out.camera_tokens, ref}};
  ctx->run(key, use_graphs(ctx), [&] { ctx->da3->forward(images, V, H, W, out, ref, ctx->hooks); });
}

// Known cameras: host [V, 4] (fx, fy, cx, cy) -> device [V, 5] with a known flag (fx and fy
// finite and > 0; other views keep the unknown-camera path, model.rs:103). NULL when no view
// is known. Copied before the (possibly graph-replayed) forward, which reads it from device
// memory.
const double* stage_cameras(Context* ctx, const double* intrinsics, int V) {
  if (!intrinsics) return nullptr;
  std::vector<double> cam(size_t(V) * 5, 0.0);
  bool any = false;
  for (int v = 0; v < V; ++v) {
    const double* k = intrinsics + 4 * v;
    const bool known = std::isfinite(k[0]) && std::isfinite(k[1]) && std::isfinite(k[2]) && std::isfinite(k[3]) &&
                       k[0] > 0 && k[1] > 0;
    if (known) {
      for (int j = 0; j < 4; ++j) cam[size_t(v) * 5 + j] = k[j];
      cam[size_t(v) * 5 + 4] = 1.0;
      any = true;
    } else {
      cam[size_t(v) * 5 + 0] = cam[size_t(v) * 5 + 1] = 1.0;  // finite placeholders, never added
    }
  }
  if (!any) return nullptr;
  double* d = static_cast<double*>(staging(ctx, 18, cam.size() * sizeof(double)));
  SPLAT_HIP(hipMemcpyAsync(d, cam.data(), cam.size() * sizeof(double), hipMemcpyHostToDevice, ctx->stream));
  SPLAT_HIP(hipStreamSynchronize(ctx->stream));
  return d;
}

void ma_device(Context* ctx, const float* images, int V, int H, int W, const splat_ma_out& out, float* tokens,
               bool encoder_only, const double* intrinsics = nullptr) {
  SPLAT_CHECK(ctx->ma != nullptr, NOT_LOADED, "no MapAnything model loaded");
  check_images(images, V, H, W);
  ctx->ma->prepare(V, H, W);
  const double* cam = encoder_only ? nullptr : stage_cameras(ctx, intrinsics, V);
  Context::GraphKey key{encoder_only ? 2 : (cam ? 3 : 1), V, H, W, images,
                        {out.raw, out.quaternion, out.translation, out.scale, out.points, out.conf, out.mask, tokens, cam}};
  ctx->run(key, use_graphs(ctx), [&] { ctx->ma->forward(images, V, H, W, out, tokens, encoder_only, ctx->hooks, cam); });
}

void load_ma(Context* ctx, SafeTensors& st, const splat_ma_spec* spec, int dtype) {
  splat_ma_spec s;
  if (spec) s = *spec;
  else splat_ma_reference_spec(&s);
  const int dt = model_dtype(dtype);
  ctx->clear_graphs();
  ctx->ma.reset();
  ctx->ma = std::make_unique<MaModel>(*ctx, st, s, dt);
}

void load_da3(Context* ctx, SafeTensors& st, int variant, int dtype, int strategy) {
  const int dt = model_dtype(dtype);
  ctx->clear_graphs();
  ctx->da3.reset();
  ctx->da3 = std::make_unique<Da3Model>(*ctx, st, variant, dt, strategy);
}

AttnArgs attention_args(int dtype, const void* qkv, void* out, int S, int L, int heads) {
  AttnArgs a;
  a.dt = model_dtype(dtype);
  const size_t es = dtype_size(a.dt);
  a.q = qkv;
  a.k = static_cast<const char*>(qkv) + size_t(heads) * 64 * es;
  a.v = static_cast<const char*>(qkv) + size_t(heads) * 128 * es;
  a.ld = 3L * heads * 64;
  a.o = out;
  a.ldo = long(heads) * 64;
  a.L = L;
  a.heads = heads;
  a.seqs = S;
  a.seq_stride = L;
  return a;
}
template <typename T>
void d2h(Context* ctx, T* host, const void* dev, size_t count) {
  if (host) SPLAT_HIP(hipMemcpyAsync(host, dev, count * sizeof(T), hipMemcpyDeviceToHost, ctx->stream));
}

}  // namespace

extern "C" {

int splat_create(int hip_device, splat_ctx** out) {
  if (!out) return BAD_ARGUMENT;
  *out = nullptr;
  try {
    *out = reinterpret_cast<splat_ctx*>(new Context(hip_device));
    return OK;
  } catch (const Error& e) {
    g_create_error = e.what();
    return e.code;
  } catch (const std::exception& e) {
    g_create_error = e.what();
    return HIP_ERROR;
  }
}

void splat_destroy(splat_ctx* ctx) {
  if (!ctx) return;
  delete C(ctx);
}

const char* splat_last_error(const splat_ctx* ctx) {
  if (!ctx) return g_create_error.c_str();
  return reinterpret_cast<const Context*>(ctx)->last_error.c_str();
}

void* splat_stream(splat_ctx* ctx) { return ctx ? static_cast<void*>(C(ctx)->stream) : nullptr; }

int splat_synchronize(splat_ctx* ctx) {
  return guard(C(ctx), [&] { SPLAT_HIP(hipStreamSynchronize(C(ctx)->stream)); });
}

int splat_set_graphs(splat_ctx* ctx, int enable) {
  return guard(C(ctx), [&] {
    C(ctx)->graphs = enable != 0;
    if (!enable) C(ctx)->clear_graphs();
  });
}

int splat_set_debug_taps(splat_ctx* ctx, splat_tap_fn fn, void* user) {
  return guard(C(ctx), [&] {
    C(ctx)->hooks.tap = fn;
    C(ctx)->hooks.tap_user = user;
  });
}

int splat_set_branch_taps(splat_ctx* ctx, splat_branch_tap_fn fn, void* user) {
  return guard(C(ctx), [&] {
    C(ctx)->hooks.branch_tap = fn;
    C(ctx)->hooks.branch_user = user;
  });
}

int splat_load_da3(splat_ctx* ctx, const char* path, int variant, int dtype, int ref_strategy) {
  return guard(C(ctx), [&] {
    SPLAT_CHECK(path != nullptr, BAD_ARGUMENT, "path is NULL");
    SafeTensors st;
    st.open_file(path);
    load_da3(C(ctx), st, variant, dtype, ref_strategy);
  });
}

int splat_load_da3_bytes(splat_ctx* ctx, const uint8_t* bytes, size_t len, int variant, int dtype, int ref_strategy) {
  return guard(C(ctx), [&] {
    SPLAT_CHECK(bytes != nullptr, BAD_ARGUMENT, "bytes is NULL");
    SafeTensors st;
    st.open_bytes(bytes, len);
    load_da3(C(ctx), st, variant, dtype, ref_strategy);
  });
}

int splat_da3_forward_raw_device(splat_ctx* ctx, const float* images, int V, int H, int W, splat_da3_out* out,
                                 int32_t* ref_view_device) {
  return guard(C(ctx), [&] {
    SPLAT_CHECK(out != nullptr, BAD_ARGUMENT, "out is NULL");
    da3_device(C(ctx), images, V, H, W, *out, ref_view_device);
  });
}

int splat_da3_forward_raw(splat_ctx* ctx, const float* images, int V, int H, int W, splat_progress_fn progress,
                          void* user, splat_da3_out* out) {
  Context* c = C(ctx);
  int rc = guard(c, [&] {
    SPLAT_CHECK(out != nullptr, BAD_ARGUMENT, "out is NULL");
    check_images(images, V, H, W);
    SPLAT_CHECK(c->da3 != nullptr, NOT_LOADED, "no Depth Anything 3 model loaded");
    const size_t R = H / 14, Cc = W / 14, hw = size_t(H) * W, d = c->da3->dim();
    const size_t img = size_t(V) * 3 * hw;
    float* d_img = static_cast<float*>(staging(c, 0, img * 4));
    splat_da3_out dev{};
    dev.depth = static_cast<float*>(staging(c, 1, V * hw * 4));
    dev.depth_conf = static_cast<float*>(staging(c, 2, V * hw * 4));
    dev.ray_logits = out->ray_logits ? static_cast<float*>(staging(c, 3, V * 7 * 64 * R * Cc * 4)) : nullptr;
    dev.pose_encoding = static_cast<float*>(staging(c, 4, V * 9 * 4));
    dev.camera_tokens = out->camera_tokens ? static_cast<float*>(staging(c, 5, V * 2 * d * 4)) : nullptr;
    int32_t* d_ref = static_cast<int32_t*>(staging(c, 6, 4));
    SPLAT_HIP(hipMemcpyAsync(d_img, images, img * 4, hipMemcpyHostToDevice, c->stream));
    c->hooks.progress = progress;
    c->hooks.progress_user = user;
    try {
      da3_device(c, d_img, V, H, W, dev, d_ref);
    } catch (...) {
      c->hooks.progress = nullptr;
      throw;
    }
    c->hooks.progress = nullptr;
    SPLAT_CHECK(out->depth && out->depth_conf && out->pose_encoding, BAD_ARGUMENT, "missing output buffers");
    d2h(c, out->depth, dev.depth, V * hw);
    d2h(c, out->depth_conf, dev.depth_conf, V * hw);
    d2h(c, out->ray_logits, dev.ray_logits, V * 7 * 64 * R * Cc);
    d2h(c, out->pose_encoding, dev.pose_encoding, V * 9);
    d2h(c, out->camera_tokens, dev.camera_tokens, V * 2 * d);
    int32_t ref = 0;
    SPLAT_HIP(hipMemcpyAsync(&ref, d_ref, 4, hipMemcpyDeviceToHost, c->stream));
    SPLAT_HIP(hipStreamSynchronize(c->stream));
    out->reference_view = ref;
  });
  if (rc != OK) return rc;
  // depthanything3-rs/src/model.rs:139-146: finite and positive depth, finite confidence
  for (size_t i = 0; i < size_t(V) * H * W; ++i) {
    if (!std::isfinite(out->depth[i]) || !(out->depth[i] > 0.f) || !std::isfinite(out->depth_conf[i])) {
      c->last_error = "view " + std::to_string(i / (size_t(H) * W)) + ": depth or confidence is not finite and positive";
      return NONFINITE;
    }
  }
  return OK;
}

void splat_ma_reference_spec(splat_ma_spec* s) {
  if (!s) return;
  // mapanything-rs/src/dinov2.rs:8-10, vit_block.rs:42-44, info_sharing.rs:12-14, dpt.rs:10-14, heads.rs:9-15
  *s = splat_ma_spec{1536, 24, 24, 1, 4096, 1536, 24, 16, 1, 4096, {7, 11, 15}, {96, 192, 384, 768}, 256, 784, 196};
}

int splat_load_mapanything(splat_ctx* ctx, const char* path, const splat_ma_spec* spec, int dtype) {
  return guard(C(ctx), [&] {
    SPLAT_CHECK(path != nullptr, BAD_ARGUMENT, "path is NULL");
    SafeTensors st;
    st.open_file(path);
    load_ma(C(ctx), st, spec, dtype);
  });
}

int splat_load_mapanything_bytes(splat_ctx* ctx, const uint8_t* bytes, size_t len, const splat_ma_spec* spec, int dtype) {
  return guard(C(ctx), [&] {
    SPLAT_CHECK(bytes != nullptr, BAD_ARGUMENT, "bytes is NULL");
    SafeTensors st;
    st.open_bytes(bytes, len);
    load_ma(C(ctx), st, spec, dtype);
  });
}

int splat_ma_forward_device(splat_ctx* ctx, const float* images, int V, int H, int W, const double* intrinsics,
                            splat_ma_out* out) {
  return guard(C(ctx), [&] {
    SPLAT_CHECK(out != nullptr, BAD_ARGUMENT, "out is NULL");
    ma_device(C(ctx), images, V, H, W, *out, nullptr, false, intrinsics);
  });
}

int splat_ma_forward(splat_ctx* ctx, const float* images, int V, int H, int W, const double* intrinsics,
                     splat_ma_out* out) {
  Context* c = C(ctx);
  return guard(c, [&] {
    SPLAT_CHECK(out != nullptr, BAD_ARGUMENT, "out is NULL");
    check_images(images, V, H, W);
    SPLAT_CHECK(c->ma != nullptr, NOT_LOADED, "no MapAnything model loaded");
    const size_t hw = size_t(H) * W, img = size_t(V) * 3 * hw;
    float* d_img = static_cast<float*>(staging(c, 10, img * 4));
    splat_ma_out dev{};
    dev.raw = out->raw ? static_cast<float*>(staging(c, 11, V * 6 * hw * 4)) : nullptr;
    dev.quaternion = static_cast<float*>(staging(c, 12, V * 4 * 4));
    dev.translation = static_cast<float*>(staging(c, 13, V * 3 * 4));
    dev.scale = static_cast<float*>(staging(c, 14, 4));
    dev.points = out->points ? static_cast<float*>(staging(c, 15, V * hw * 3 * 4)) : nullptr;
    dev.conf = out->conf ? static_cast<float*>(staging(c, 16, V * hw * 4)) : nullptr;
    dev.mask = out->mask ? static_cast<uint8_t*>(staging(c, 17, V * hw)) : nullptr;
    SPLAT_HIP(hipMemcpyAsync(d_img, images, img * 4, hipMemcpyHostToDevice, c->stream));
    ma_device(c, d_img, V, H, W, dev, nullptr, false, intrinsics);
    d2h(c, out->raw, dev.raw, V * 6 * hw);
    d2h(c, out->quaternion, dev.quaternion, V * 4);
    d2h(c, out->translation, dev.translation, V * 3);
    d2h(c, out->scale, dev.scale, 1);
    d2h(c, out->points, dev.points, V * hw * 3);
    d2h(c, out->conf, dev.conf, V * hw);
    d2h(c, out->mask, dev.mask, V * hw);
    SPLAT_HIP(hipStreamSynchronize(c->stream));
  });
}

int splat_ma_encode_device(splat_ctx* ctx, const float* images, int V, int H, int W, float* tokens) {
  return guard(C(ctx), [&] {
    SPLAT_CHECK(tokens != nullptr, BAD_ARGUMENT, "tokens is NULL");
    splat_ma_out none{};
    ma_device(C(ctx), images, V, H, W, none, tokens, true);
  });
}

// A single GEMM outside a forward: a dry pass sizes its split-K workspace first.
static void gemm_now(Context* c, const GemmArgs& g) {
  Exec dry = c->ex;
  dry.dry = true;
  gemm(dry, g);
  if (c->reserve_workspace()) c->clear_graphs();
  gemm(c->ex, g);
}

int splat_kernel_gemm(splat_ctx* ctx, int dtype, const void* A, int M, int K, const void* W, int N, int ldw,
                      const float* bias, int act, void* out, int out_f32) {
  return guard(C(ctx), [&] {
    SPLAT_CHECK(act >= 0 && act <= 2, BAD_ARGUMENT, "act");
    GemmArgs g;
    g.dt = model_dtype(dtype);
    g.M = M;
    g.N = N;
    g.K = K;
    g.A = A;
    g.lda = K;
    g.W = W;
    g.ldw = ldw;
    g.bias = bias;
    g.act = act;
    g.out = out;
    g.ldc = N;
    g.out_f32 = out_f32;
    gemm_now(C(ctx), g);
  });
}

int splat_kernel_gemm_ln(splat_ctx* ctx, int dtype, const void* A, int M, int K, const void* W, int N, int ldw,
                         const float* bias, int act, const float* ln_in, const float* c1, float eps,
                         const float* gamma, const float* res, float* ln_out, void* copy, int group, void* out,
                         int out_f32) {
  return guard(C(ctx), [&] {
    SPLAT_CHECK(act >= 0 && act <= 2, BAD_ARGUMENT, "act");
    SPLAT_CHECK(group == 64 || group == 128, BAD_ARGUMENT, "statistics group: 64 or 128 columns");
    SPLAT_CHECK(!ln_in || K % group == 0, BAD_ARGUMENT, "folded LayerNorm: K must be a multiple of the group");
    SPLAT_CHECK(!(ln_in && res), BAD_ARGUMENT, "a folded LayerNorm has no residual epilogue");
    SPLAT_CHECK(!res || out_f32, BAD_ARGUMENT, "residual epilogue: fp32 output");
    SPLAT_CHECK(!ln_out || res, BAD_ARGUMENT, "row statistics come from the residual epilogue");
    GemmArgs g;
    g.dt = model_dtype(dtype);
    g.M = M;
    g.N = N;
    g.K = K;
    g.A = A;
    g.lda = K;
    g.W = W;
    g.ldw = ldw;
    g.bias = bias;
    g.act = act;
    g.out = out;
    g.ldc = N;
    g.out_f32 = out_f32;
    if (ln_in) {
      g.ln_in = ln_in;
      g.ln_parts = K / group;
      g.ln_c1 = c1;
      g.ln_eps = eps;
    }
    if (res) {
      g.gamma = gamma;
      g.res = res;
      g.ldres = N;
      g.res_f32 = 1;
      g.ln_out = ln_out;
      g.ln_group = group;
      g.ln_copy = ln_out ? copy : nullptr;
    }
    gemm_now(C(ctx), g);
  });
}

int splat_kernel_ln_stats(splat_ctx* ctx, const float* x, int rows, int n, int group, float* stats, int dtype,
                          void* copy) {
  return guard(C(ctx), [&] {
    ln_stats(C(ctx)->ex, x, n, rows, n, group, stats, model_dtype(dtype), copy);
  });
}

int splat_kernel_attention_noalloc(splat_ctx* ctx, int dtype, const void* qkv, void* out, int S, int L, int heads) {
  return guard(C(ctx), [&] {
    Context* c = C(ctx);
    const AttnArgs a = attention_args(dtype, qkv, out, S, L, heads);
    // the same kernels and key-slice plan as splat_kernel_attention, with the partials in this
    // device's static scratch instead of the context's workspace; a launch whose partials would
    // not fit runs as one key slice (no partials), as attention() does on an unsized workspace.
    // No profiling records (their events are created per launch).
    SPLAT_CHECK(c->attn_scratch != nullptr, HIP_ERROR, "attention scratch: not set up");
    Workspace ws;
    ws.ptr = c->attn_scratch;
    ws.cap = ATTN_SCRATCH_BYTES;
    Exec e = c->ex;
    e.ws = &ws;
    e.prof = nullptr;
    attention_scratch_ordered(c->device, e.stream, [&] { attention(e, a); });
  });
}

int splat_kernel_attention(splat_ctx* ctx, int dtype, const void* qkv, void* out, int S, int L, int heads) {
  return guard(C(ctx), [&] {
    const AttnArgs a = attention_args(dtype, qkv, out, S, L, heads);
    Context* c = C(ctx);
    Exec dry = c->ex;  // a dry pass sizes the key-split partials first
    dry.dry = true;
    attention(dry, a);
    if (c->reserve_workspace()) c->clear_graphs();
    attention(c->ex, a);
  });
}

int splat_profile_begin(splat_ctx* ctx) {
  return guard(C(ctx), [&] {
    Context* c = C(ctx);
    if (!c->profiler) c->profiler = std::make_unique<Profiler>();
    c->ex.prof = c->profiler.get();
  });
}

int splat_profile_end(splat_ctx* ctx, splat_kernel_stat* stats, int max, int* count) {
  return guard(C(ctx), [&] {
    Context* c = C(ctx);
    SPLAT_CHECK(c->profiler != nullptr, BAD_ARGUMENT, "profiling was not started");
    SPLAT_HIP(hipStreamSynchronize(c->stream));
    std::map<std::string, splat_kernel_stat> agg;
    for (auto& r : c->profiler->recs) {
      float ms = 0.f;
      SPLAT_HIP(hipEventElapsedTime(&ms, r.e0, r.e1));
      auto& s = agg[r.name];
      s.launches += 1;
      s.ms += ms;
      s.flops += r.flops;
      s.bytes += r.bytes;
      (void)hipEventDestroy(r.e0);
      (void)hipEventDestroy(r.e1);
    }
    c->profiler->recs.clear();
    c->ex.prof = nullptr;
    std::vector<std::pair<std::string, splat_kernel_stat>> v(agg.begin(), agg.end());
    std::sort(v.begin(), v.end(), [](auto& a, auto& b) { return a.second.ms > b.second.ms; });
    int n = 0;
    for (auto& kv : v) {
      if (n >= max || !stats) break;
      splat_kernel_stat s = kv.second;
      std::snprintf(s.name, sizeof(s.name), "%s", kv.first.c_str());
      stats[n++] = s;
    }
    if (count) *count = n;
  });
}

int splat_kernel_conv2d(splat_ctx* ctx, int dtype, const void* in, int V, int H, int W, int Cin, const void* w,
                        int Cout, int ldw, int ks, int stride, const float* bias, int relu_in, int act,
                        const void* res, void* out) {
  return guard(C(ctx), [&] {
    SPLAT_CHECK(ks == 1 || ks == 3, BAD_ARGUMENT, "kernel size must be 1 or 3");
    Conv c;
    c.cout = Cout;
    c.cin = Cin;
    c.ks = ks;
    c.lin.w = const_cast<void*>(w);
    c.lin.ldw = ldw;
    c.lin.N = Cout;
    c.lin.K = ks * ks * Cin;
    c.lin.b = const_cast<float*>(bias);
    const int dt = model_dtype(dtype);
    GemmArgs g = conv_args(c, dt, in, V, H, W, stride, out);
    g.relu_in = relu_in;
    g.act = act;
    g.res = res;
    g.ldres = Cout;
    gemm_now(C(ctx), g);
  });
}

int splat_kernel_conv_transpose2d(splat_ctx* ctx, int dtype, const void* in, int V, int R, int Cc, int Cin,
                                  const void* w, int Cout, int ldw, int s, const float* bias, void* out) {
  return guard(C(ctx), [&] {
    Lin l;
    l.w = const_cast<void*>(w);
    l.ldw = ldw;
    l.N = s * s * Cout;
    l.K = Cin;
    l.b = const_cast<float*>(bias);
    GemmArgs u = lin_args(l, model_dtype(dtype), in, Cin, V * R * Cc, out, 0);
    u.store = STORE_CONVT;
    u.V = V;
    u.ct_s = s;
    u.ct_R = R;
    u.ct_C = Cc;
    u.ct_Cout = Cout;
    gemm_now(C(ctx), u);
  });
}

int splat_kernel_resize_bilinear(splat_ctx* ctx, int dtype, const void* in, int V, int Hi, int Wi, int Cc, void* out,
                                 int Ho, int Wo) {
  return guard(C(ctx), [&] {
    resize_bilinear(C(ctx)->ex, model_dtype(dtype), in, V, Hi, Wi, Cc, out, Ho, Wo, Ho, Wo, nullptr, 0);
  });
}

int splat_kernel_reconstruct(splat_ctx* ctx, int V, int H, int W, const float* depth, const float* pose_encoding,
                             const float* points_in_camera, const float* quaternion, const float* translation,
                             const float* conf, const uint8_t* mask, const uint8_t* foreground, double* cameras,
                             float* points, float* conf_out) {
  Context* c = C(ctx);
  return guard(c, [&] {
    SPLAT_CHECK(V > 0 && H > 0 && W > 0 && conf && cameras && points && conf_out, BAD_ARGUMENT, "geometry args");
    const size_t px = size_t(V) * H * W;
    float* d_conf0 = static_cast<float*>(staging(c, 21, px * 4));
    double* d_fit = depth ? nullptr : static_cast<double*>(staging(c, 24, size_t(V) * 4 * 8));
    reconstruct_geometry(c->ex, V, H, W, depth, pose_encoding, points_in_camera, quaternion, translation, conf, mask,
                         foreground, cameras, d_fit, d_conf0, points, conf_out);
  });
}

int splat_to_model_input(splat_ctx* ctx, const uint8_t* rgba, int V, int H, int W, float* images,
                         uint8_t* foreground) {
  Context* c = C(ctx);
  return guard(c, [&] {
    SPLAT_CHECK(rgba && images && V > 0 && H > 0 && W > 0, BAD_ARGUMENT, "to_model_input args");
    const size_t px = size_t(V) * H * W;
    uint8_t* d = static_cast<uint8_t*>(staging(c, 26, px * 4));
    SPLAT_HIP(hipMemcpyAsync(d, rgba, px * 4, hipMemcpyHostToDevice, c->stream));
    model_input(*c, d, V, H, W, images, foreground);
  });
}

int splat_resize_rgba8(splat_ctx* ctx, const uint8_t* src, int width, int height, uint8_t* dst, int new_width,
                       int new_height, int filter) {
  Context* c = C(ctx);
  return guard(c, [&] {
    SPLAT_CHECK(src && dst && width > 0 && height > 0 && new_width > 0 && new_height > 0, BAD_ARGUMENT, "resize args");
    uint8_t* s = static_cast<uint8_t*>(staging(c, 47, size_t(width) * height * 4));
    uint8_t* d = static_cast<uint8_t*>(staging(c, 48, size_t(new_width) * new_height * 4));
    SPLAT_HIP(hipMemcpyAsync(s, src, size_t(width) * height * 4, hipMemcpyHostToDevice, c->stream));
    resize_device(*c, s, width, height, d, new_width, new_height, filter);
    SPLAT_HIP(hipMemcpyAsync(dst, d, size_t(new_width) * new_height * 4, hipMemcpyDeviceToHost, c->stream));
    SPLAT_HIP(hipStreamSynchronize(c->stream));
  });
}

int splat_da3_input_size(int width, int height, int* bounded_width, int* bounded_height, int* out_width,
                         int* out_height) {
  return guard_free([&] {
    int bw, bh, w, h;
    da3_model_input_size(width, height, bw, bh, w, h);
    if (bounded_width) *bounded_width = bw;
    if (bounded_height) *bounded_height = bh;
    if (out_width) *out_width = w;
    if (out_height) *out_height = h;
  });
}

int splat_ma_input_size(int n, const int* widths, const int* heights, int* out_width, int* out_height) {
  return guard_free([&] {
    int w, h;
    ma_input_size(n, widths, heights, w, h);
    if (out_width) *out_width = w;
    if (out_height) *out_height = h;
  });
}

int splat_da3_model_inputs(splat_ctx* ctx, int n, const uint8_t* const* rgba, const int* widths, const int* heights,
                           float* images, uint8_t* foreground, int* out_height, int* out_width) {
  Context* c = C(ctx);
  return guard(c, [&] {
    int H, W;
    da3_model_inputs(*c, n, rgba, widths, heights, images, foreground, H, W);
    if (out_height) *out_height = H;
    if (out_width) *out_width = W;
  });
}

int splat_ma_model_inputs(splat_ctx* ctx, int n, const uint8_t* const* rgba, const int* widths, const int* heights,
                          float* images, uint8_t* foreground, int* out_height, int* out_width) {
  Context* c = C(ctx);
  return guard(c, [&] {
    int H, W;
    ma_model_inputs(*c, n, rgba, widths, heights, images, foreground, H, W);
    if (out_height) *out_height = H;
    if (out_width) *out_width = W;
  });
}

// --- post-forward reconstruction ---------------------------------------------------------------

namespace {

void recon_outputs(Context* c, int V, int H, int W, const double* d_cam, const float* d_points, const float* d_conf,
                   const float* d_depth, int depth_stride, splat_recon_out* out) {
  const size_t px = size_t(V) * H * W;
  d2h(c, out->points, d_points, px * 3);
  d2h(c, out->conf, d_conf, px);
  std::vector<double> cam(size_t(V) * 16);
  SPLAT_HIP(hipMemcpyAsync(cam.data(), d_cam, cam.size() * 8, hipMemcpyDeviceToHost, c->stream));
  std::vector<float> dep;
  if (out->depth) {
    dep.resize((px - 1) * depth_stride + 1);  // the z of the last point ends the buffer
    SPLAT_HIP(hipMemcpyAsync(dep.data(), d_depth, dep.size() * 4, hipMemcpyDeviceToHost, c->stream));
  }
  SPLAT_HIP(hipStreamSynchronize(c->stream));
  for (int v = 0; v < V; ++v) {
    const double* k = cam.data() + size_t(v) * 16;
    if (out->rotation) std::memcpy(out->rotation + size_t(v) * 9, k, 9 * 8);
    if (out->translation) std::memcpy(out->translation + size_t(v) * 3, k + 9, 3 * 8);
    if (out->focal) std::memcpy(out->focal + size_t(v) * 2, k + 12, 2 * 8);
    if (out->principal_point) std::memcpy(out->principal_point + size_t(v) * 2, k + 14, 2 * 8);
  }
  if (out->depth)
    for (size_t i = 0; i < px; ++i) out->depth[i] = dep[i * depth_stride];
}

const uint8_t* stage_foreground(Context* c, const uint8_t* fg, size_t px) {
  if (!fg) return nullptr;
  uint8_t* d = static_cast<uint8_t*>(staging(c, 25, px));
  SPLAT_HIP(hipMemcpyAsync(d, fg, px, hipMemcpyHostToDevice, c->stream));
  return d;
}

}  // namespace

int splat_da3_reconstruct(splat_ctx* ctx, const float* images, int V, int H, int W, const uint8_t* foreground,
                          splat_recon_out* out) {
  Context* c = C(ctx);
  bool finite = true;
  int rc = guard(c, [&] {
    SPLAT_CHECK(out != nullptr && out->points && out->conf, BAD_ARGUMENT, "points and conf are required");
    check_images(images, V, H, W);
    SPLAT_CHECK(c->da3 != nullptr, NOT_LOADED, "no Depth Anything 3 model loaded");
    const size_t hw = size_t(H) * W, px = size_t(V) * hw;
    float* d_img = static_cast<float*>(staging(c, 0, size_t(V) * 3 * hw * 4));
    splat_da3_out dev{};
    dev.depth = static_cast<float*>(staging(c, 1, px * 4));
    dev.depth_conf = static_cast<float*>(staging(c, 2, px * 4));
    dev.pose_encoding = static_cast<float*>(staging(c, 4, V * 9 * 4));
    int32_t* d_ref = static_cast<int32_t*>(staging(c, 6, 4));
    double* d_cam = static_cast<double*>(staging(c, 20, size_t(V) * 16 * 8));
    float* d_conf0 = static_cast<float*>(staging(c, 21, px * 4));
    float* d_points = static_cast<float*>(staging(c, 22, px * 12));
    float* d_conf = static_cast<float*>(staging(c, 23, px * 4));
    SPLAT_HIP(hipMemcpyAsync(d_img, images, px * 3 * 4, hipMemcpyHostToDevice, c->stream));
    const uint8_t* d_fg = stage_foreground(c, foreground, px);
    da3_device(c, d_img, V, H, W, dev, d_ref);
    reconstruct_geometry(c->ex, V, H, W, dev.depth, dev.pose_encoding, nullptr, nullptr, nullptr, dev.depth_conf,
                         nullptr, d_fg, d_cam, nullptr, d_conf0, d_points, d_conf);
    int32_t ref = 0;
    SPLAT_HIP(hipMemcpyAsync(&ref, d_ref, 4, hipMemcpyDeviceToHost, c->stream));
    std::vector<float> pose(size_t(V) * 9), depth(px);
    SPLAT_HIP(hipMemcpyAsync(pose.data(), dev.pose_encoding, pose.size() * 4, hipMemcpyDeviceToHost, c->stream));
    SPLAT_HIP(hipMemcpyAsync(depth.data(), dev.depth, px * 4, hipMemcpyDeviceToHost, c->stream));
    recon_outputs(c, V, H, W, d_cam, d_points, d_conf, dev.depth, 1, out);
    out->reference_view = ref;
    // DepthAnything3::forward's asserts (model.rs:139-146): finite positive depth, finite camera
    for (float d : depth) finite = finite && std::isfinite(d) && d > 0.f;
    for (float e : pose) finite = finite && std::isfinite(e);
  });
  if (rc != OK) return rc;
  if (!finite) {
    c->last_error = "depth or camera is not finite and positive (outputs written)";
    return NONFINITE;
  }
  return OK;
}

int splat_ma_reconstruct(splat_ctx* ctx, const float* images, int V, int H, int W, const double* intrinsics,
                         const uint8_t* foreground, splat_recon_out* out) {
  Context* c = C(ctx);
  return guard(c, [&] {
    SPLAT_CHECK(out != nullptr && out->points && out->conf, BAD_ARGUMENT, "points and conf are required");
    check_images(images, V, H, W);
    SPLAT_CHECK(c->ma != nullptr, NOT_LOADED, "no MapAnything model loaded");
    const size_t hw = size_t(H) * W, px = size_t(V) * hw;
    float* d_img = static_cast<float*>(staging(c, 10, size_t(V) * 3 * hw * 4));
    splat_ma_out dev{};
    dev.quaternion = static_cast<float*>(staging(c, 12, V * 4 * 4));
    dev.translation = static_cast<float*>(staging(c, 13, V * 3 * 4));
    dev.scale = static_cast<float*>(staging(c, 14, 4));
    dev.points = static_cast<float*>(staging(c, 15, px * 12));
    dev.conf = static_cast<float*>(staging(c, 16, px * 4));
    dev.mask = static_cast<uint8_t*>(staging(c, 17, px));
    double* d_cam = static_cast<double*>(staging(c, 20, size_t(V) * 16 * 8));
    float* d_conf0 = static_cast<float*>(staging(c, 21, px * 4));
    float* d_points = static_cast<float*>(staging(c, 22, px * 12));
    float* d_conf = static_cast<float*>(staging(c, 23, px * 4));
    double* d_fit = static_cast<double*>(staging(c, 24, size_t(V) * 4 * 8));
    SPLAT_HIP(hipMemcpyAsync(d_img, images, px * 3 * 4, hipMemcpyHostToDevice, c->stream));
    const uint8_t* d_fg = stage_foreground(c, foreground, px);
    ma_device(c, d_img, V, H, W, dev, nullptr, false, intrinsics);
    reconstruct_geometry(c->ex, V, H, W, nullptr, nullptr, dev.points, dev.quaternion, dev.translation, dev.conf,
                         dev.mask, d_fg, d_cam, d_fit, d_conf0, d_points, d_conf);
    recon_outputs(c, V, H, W, d_cam, d_points, d_conf, dev.points + 2, 3, out);
    out->reference_view = 0;
  });
}

int splat_ma_encode(splat_ctx* ctx, const float* images, int V, int H, int W, float* tokens) {
  Context* c = C(ctx);
  return guard(c, [&] {
    SPLAT_CHECK(tokens != nullptr, BAD_ARGUMENT, "tokens is NULL");
    check_images(images, V, H, W);
    SPLAT_CHECK(c->ma != nullptr, NOT_LOADED, "no MapAnything model loaded");
    const size_t hw = size_t(H) * W, img = size_t(V) * 3 * hw;
    const size_t nt = size_t(V) * (1 + (H / 14) * (W / 14)) * c->ma->spec().enc_dim;
    float* d_img = static_cast<float*>(staging(c, 20, img * 4));
    float* d_tok = static_cast<float*>(staging(c, 21, nt * 4));
    SPLAT_HIP(hipMemcpyAsync(d_img, images, img * 4, hipMemcpyHostToDevice, c->stream));
    splat_ma_out none{};
    ma_device(c, d_img, V, H, W, none, d_tok, true);
    d2h(c, tokens, d_tok, nt);
    SPLAT_HIP(hipStreamSynchronize(c->stream));
  });
}

}  // extern "C"
