// Depth Anything 3: weights (depthanything3-rs/src/{backbone,vit_block,dpt,camera_head}.rs
// ::new) and the forward of DepthAnything3::forward_raw (model.rs:105-123), all views batched
// through every stage.
#include <algorithm>
#include <cstring>

#include "runtime.h"

namespace splat {

namespace {
constexpr int PATCH = 14;
constexpr int KPATCH = 640;      // 3*14*14 = 588 patch values, zero-padded to 64
constexpr int OUT_HIDDEN = 32;   // depthanything3-rs/src/dpt.rs:17
}  // namespace

int Da3Spec::hidden() const { return swiglu ? (dim * 4 * 2 / 3 + 7) / 8 * 8 : 4 * dim; }

// depthanything3-rs/src/variant.rs:59-113
Da3Spec da3_variant_spec(int variant) {
  switch (variant) {
    case 0: return {384, 6, 12, 0, 4, {5, 7, 9, 11}, 64, {48, 96, 192, 384}};
    case 1: return {768, 12, 12, 0, 4, {5, 7, 9, 11}, 128, {96, 192, 384, 768}};
    case 2: return {1024, 16, 24, 0, 8, {11, 15, 19, 23}, 256, {256, 512, 1024, 1024}};
    case 3: return {1536, 24, 40, 1, 13, {19, 27, 33, 39}, 256, {256, 512, 1024, 1024}};
  }
  throw Error(BAD_ARGUMENT, "unknown DA3 variant " + std::to_string(variant));
}

Da3Model::Da3Model(Context& ctx, const SafeTensors& st, int variant, int dt, int strategy)
    : ctx_(ctx), spec_(da3_variant_spec(variant)), dt_(dt), strategy_(strategy) {
  SPLAT_CHECK(strategy >= 0 && strategy <= 2, BAD_ARGUMENT, "unknown reference-view strategy");
  Loader L(ctx, st, dt, "model.");
  const int d = spec_.dim, F = spec_.head_features, hin = 2 * d;
  const std::string b = "backbone.pretrained";
  {
    auto w = L.host(b + ".patch_embed.proj.weight", {d, 3, PATCH, PATCH});
    float* bias = L.vec(b + ".patch_embed.proj.bias", {d});
    patch_ = L.pack(w, d, 3 * PATCH * PATCH, bias, dt);
  }
  cls_ = L.vec(b + ".cls_token", {1, 1, d});
  camera_ = L.vec(b + ".camera_token", {1, 2, d});
  pos_host_ = L.host(b + ".pos_embed", {1, 1 + 37 * 37, d});
  norm_ = L.ln(b + ".norm", d);
  for (int i = 0; i < spec_.depth; ++i)
    blocks_.push_back(L.block(b + ".blocks." + std::to_string(i), d, spec_.hidden(), spec_.swiglu, i >= spec_.alt_start));
  // dense head (depthanything3-rs/src/dpt.rs:191-242)
  head_norm_ = L.ln("head.norm", hin);
  const int* c = spec_.stage_dims;
  for (int k = 0; k < 4; ++k) {
    proj_[k] = L.conv("head.projects." + std::to_string(k), c[k], hin, 1).lin;
    rn_[k] = L.conv("head.scratch.layer" + std::to_string(k + 1) + "_rn", F, c[k], 3, false);
  }
  rs0_ = L.convt("head.resize_layers.0", c[0], c[0], 4);
  rs1_ = L.convt("head.resize_layers.1", c[1], c[1], 2);
  rs3_ = L.conv("head.resize_layers.3", c[3], c[3], 3);
  for (int level = 1; level <= 4; ++level) {
    const std::string p = "head.scratch.refinenet" + std::to_string(level);
    depth_chain_[level - 1] = load_fusion(L, p, F, level < 4);
    ray_chain_[level - 1] = load_fusion(L, p + "_aux", F, level < 4);
  }
  out_conv1_ = L.conv("head.scratch.output_conv1", F / 2, F, 3);
  oc2_0_ = L.conv("head.scratch.output_conv2.0", OUT_HIDDEN, F / 2, 3);
  oc2_2_w_ = L.vec("head.scratch.output_conv2.2.weight", {2, OUT_HIDDEN, 1, 1});
  oc2_2_b_ = L.vec("head.scratch.output_conv2.2.bias", {2});
  for (int i = 0; i < 5; ++i) {
    const int cin = i % 2 == 0 ? F : F / 2, cout = i % 2 == 0 ? F / 2 : F;
    ray_pre_[i] = L.conv("head.scratch.output_conv1_aux.3." + std::to_string(i), cout, cin, 3);
  }
  ray_out_conv_ = L.conv("head.scratch.output_conv2_aux.3.0", OUT_HIDDEN, F / 2, 3);
  ray_out_w_ = L.vec("head.scratch.output_conv2_aux.3.5.weight", {7, OUT_HIDDEN, 1, 1});
  ray_out_b_ = L.vec("head.scratch.output_conv2_aux.3.5.bias", {7});
  // camera head (depthanything3-rs/src/camera_head.rs:65-78): output layers in f32
  cam_h_[0] = L.linear("cam_dec.backbone.0", hin, hin);
  cam_h_[1] = L.linear("cam_dec.backbone.2", hin, hin);
  cam_t_ = L.linear("cam_dec.fc_t", 3, hin, true, F32);
  cam_q_ = L.linear("cam_dec.fc_qvec", 4, hin, true, F32);
  cam_f_ = L.linear("cam_dec.fc_fov.0", 2, hin, true, F32);
}

void Da3Model::prepare(int V, int H, int W) {
  (void)V;
  const int R = H / PATCH, C = W / PATCH;
  auto key = std::make_tuple(R, C);
  if (tables_.count(key)) return;
  Tables t;
  const int d = spec_.dim, F = spec_.head_features;
  auto pos = resize_pos_embed(pos_host_, d, R, C);
  t.pos = static_cast<float*>(ctx_.pool.upload(pos.data(), pos.size() * 4));
  t.npos = std::max(R, C) + 2;
  auto rope = rope_table(t.npos);
  t.rope = static_cast<float*>(ctx_.pool.upload(rope.data(), rope.size() * 4));
  const double aspect = double(W) / double(H);
  for (int k = 0; k < 4; ++k) {
    auto uv = uv_table(spec_.stage_dims[k], R, C, aspect);
    t.uv[k] = static_cast<float*>(ctx_.pool.upload(uv.data(), uv.size() * 4));
  }
  auto uvi = uv_table(F / 2, H, W, aspect);
  t.uv_img = static_cast<float*>(ctx_.pool.upload(uvi.data(), uvi.size() * 4));
  auto uvr = uv_table(F / 2, 8 * R, 8 * C, aspect);
  t.uv_ray = static_cast<float*>(ctx_.pool.upload(uvr.data(), uvr.size() * 4));
  tables_[key] = t;
}

// depthanything3-rs/src/dpt.rs:156-164: exact sizes from the next finer level, the finest
// fused at twice its size.
void Da3Model::fusion_chain(const FusionW* chain, void* const pyr[4], const int ph[4], const int pw[4], int V, void* out,
                            const Exec& ex, bool keep) {
  const int F = spec_.head_features;
  const size_t es = dtype_size(dt_);
  void* t3 = ctx_.arena.alloc(size_t(V) * ph[2] * pw[2] * F * es);
  fusion_block(ctx_, dt_, chain[3], pyr[3], nullptr, V, ph[3], pw[3], ph[2], pw[2], ph[2], pw[2], t3, &ex, keep);
  void* t2 = ctx_.arena.alloc(size_t(V) * ph[1] * pw[1] * F * es);
  fusion_block(ctx_, dt_, chain[2], t3, pyr[2], V, ph[2], pw[2], ph[1], pw[1], ph[1], pw[1], t2, &ex, keep);
  void* t1 = ctx_.arena.alloc(size_t(V) * ph[0] * pw[0] * F * es);
  fusion_block(ctx_, dt_, chain[1], t2, pyr[1], V, ph[1], pw[1], ph[0], pw[0], ph[0], pw[0], t1, &ex, keep);
  fusion_block(ctx_, dt_, chain[0], t1, pyr[0], V, ph[0], pw[0], 2 * ph[0], 2 * pw[0], 2 * ph[0], 2 * pw[0], out, &ex,
               keep);
}

void Da3Model::forward(const float* images, int V, int H, int W, const splat_da3_out& out, int32_t* ref_dev,
                       const Hooks& hooks) {
  const Exec& ex = ctx_.ex;
  Arena& ar = ctx_.arena;
  const int R = H / PATCH, C = W / PATCH, P = R * C, n = P + 1, T = V * n, d = spec_.dim;
  const int F = spec_.head_features;
  const size_t es = dtype_size(dt_);
  const Tables& tb = tables_.at(std::make_tuple(R, C));
  auto progress = [&](int stage, int block) {
    if (hooks.progress && !ex.dry) hooks.progress(stage, block, hooks.progress_user);
  };

  float* X0 = ar.alloc_t<float>(size_t(T) * d);
  float* X1 = ar.alloc_t<float>(size_t(T) * d);
  int32_t* ref = ref_dev ? ref_dev : ar.alloc_t<int32_t>(1);
  float* cam_tok = out.camera_tokens ? out.camera_tokens : ar.alloc_t<float>(size_t(V) * 2 * d);
  void* hook[4];
  for (int k = 0; k < 4; ++k) hook[k] = ar.alloc(size_t(V) * P * 2 * d * es);

  // ---- backbone (depthanything3-rs/src/backbone.rs:128-196)
  {
    const size_t mark = ar.mark();
    void* patches = ar.alloc(size_t(V) * P * KPATCH * es);
    im2col_patch(ex, dt_, images, V, H, W, patches, KPATCH);
    GemmArgs g = lin_args(patch_, dt_, patches, KPATCH, V * P, X0, d);
    g.K = KPATCH;
    g.addtab = tb.pos + d;
    g.addtab_period = P;
    g.out_f32 = 1;
    g.rm_P = P;
    g.rm_n = n;
    g.rm_off = 1;
    gemm(ex, g);
    write_class_rows(ex, X0, V, n, d, cls_, tb.pos);
    ar.release(mark);
  }
  const size_t mark = ar.mark();
  BlockScratch s;
  block_scratch(ctx_, s, dt_, T, d, spec_.hidden());
  float* cur = X0;
  float* within = X0;
  const int sel_at = std::max(spec_.alt_start - 1, 0);
  std::vector<float> tap_host;
  for (int i = 0; i < spec_.depth; ++i) {
    progress(SPLAT_STAGE_BLOCK, i);
    if (i == sel_at) {
      // Views are never reordered here: every block is equivariant to the view order, so
      // only the camera-token assignment depends on the reference view.
      const int strat = (V >= 3 && spec_.alt_start >= 1) ? strategy_ : 0;
      select_reference_view(ex, cur, V, n, d, strat, ref);
    }
    if (i == spec_.alt_start) {
      set_camera_tokens(ex, cur, V, n, d, camera_, ref);
      if (s.ln_src == cur) block_ln_refresh(ctx_, dt_, cur, V, d, s, 1, n, 0);  // the rewritten class rows
    }
    const bool across = i >= spec_.alt_start && i % 2 == 1;
    const int rope = i >= spec_.alt_start ? (across ? 2 : 1) : 0;
    float* dst = cur == within ? (cur == X0 ? X1 : X0) : cur;
    if (across) {
      block_forward(ctx_, blocks_[i], dt_, cur, dst, T, 1, T, s, rope, n, C, tb.rope, tb.npos, i);
    } else {
      block_forward(ctx_, blocks_[i], dt_, cur, dst, T, V, n, s, rope, n, C, tb.rope, tb.npos, i);
      within = dst;
    }
    cur = dst;
    if (hooks.tap && !ex.dry) {
      tap_host.resize(size_t(T) * d);
      SPLAT_HIP(hipMemcpyAsync(tap_host.data(), cur, tap_host.size() * 4, hipMemcpyDeviceToHost, ex.stream));
      SPLAT_HIP(hipStreamSynchronize(ex.stream));
      hooks.tap(i, tap_host.data(), T, d, hooks.tap_user);
    }
    for (int k = 0; k < 4; ++k)
      if (spec_.out_layers[k] == i)
        da3_hook(ex, dt_, within, cur, V, n, d, norm_.w, norm_.b, head_norm_.w, head_norm_.b, hook[k],
                 k == 3 ? cam_tok : nullptr);
  }
  ar.release(mark);

  // ---- dense head (depthanything3-rs/src/dpt.rs:256-300), all views at once
  progress(SPLAT_STAGE_DENSE_HEAD, 0);
  const int* c = spec_.stage_dims;
  const int R2 = (R - 1) / 2 + 1, C2 = (C - 1) / 2 + 1;
  const int ph[4] = {4 * R, 2 * R, R, R2}, pw[4] = {4 * C, 2 * C, C, C2};
  void* pyr[4];
  for (int k = 0; k < 4; ++k) pyr[k] = ar.alloc(size_t(V) * ph[k] * pw[k] * F * es);
  // The four hook adapters are independent until the fusion chains: levels 2 and 3 run on the
  // context's second stream while 0 and 1 run here (their convolutions each leave most CUs
  // idle). The second stream's levels are enqueued first and keep their arena memory until the
  // join.
  auto adapter = [&](int k, const Exec& e, bool keep) {
    const size_t m = ar.mark();
    void* pk = ar.alloc(size_t(V) * P * c[k] * es);
    GemmArgs g = lin_args(proj_[k], dt_, hook[k], 2 * d, V * P, pk, c[k]);
    g.addtab = tb.uv[k];
    g.addtab_period = P;
    gemm(e, g);
    const void* r = pk;
    if (k == 0 || k == 1) {
      const ConvT& ct = k == 0 ? rs0_ : rs1_;
      void* up = ar.alloc(size_t(V) * P * ct.s * ct.s * c[k] * es);
      GemmArgs u = lin_args(ct.lin, dt_, pk, c[k], V * P, up, 0);
      u.store = STORE_CONVT;
      u.V = V;
      u.ct_s = ct.s;
      u.ct_R = R;
      u.ct_C = C;
      u.ct_Cout = c[k];
      gemm(e, u);
      r = up;
    } else if (k == 3) {
      void* dn = ar.alloc(size_t(V) * R2 * C2 * c[k] * es);
      gemm(e, conv_args(rs3_, dt_, pk, V, R, C, 2, dn));
      r = dn;
    }
    gemm(e, conv_args(rn_[k], dt_, r, V, ph[k], pw[k], 1, pyr[k]));
    if (!keep) ar.release(m);
  };
  {
    const size_t madapt = ar.mark();
    const Exec ax = ctx_.fork(ex);
    adapter(3, ax, true);
    adapter(2, ax, true);
    adapter(0, ex, false);
    adapter(1, ex, false);
    ctx_.join(ex);
    ar.release(madapt);
  }
  const int FH = 8 * R, FW = 8 * C;
  {
    // The ray branch (its fusion chain and output convs) runs on the context's second stream
    // while the depth branch runs on this one; both only read the pyramid. The ray branch is
    // enqueued first and keeps all of its arena memory until the join, so nothing the depth
    // branch allocates (or hands back) overlaps memory the ray branch may still be using.
    const size_t m = ar.mark();
    const Exec rx = ctx_.fork(ex);
    void* rays = ar.alloc(size_t(V) * FH * FW * F * es);
    fusion_chain(ray_chain_, pyr, ph, pw, V, rays, rx, true);
    const void* r = rays;
    for (int i = 0; i < 5; ++i) {
      void* o = ar.alloc(size_t(V) * FH * FW * ray_pre_[i].cout * es);
      GemmArgs g = conv_args(ray_pre_[i], dt_, r, V, FH, FW, 1, o);
      if (i == 4) {
        g.addtab = tb.uv_ray;
        g.addtab_period = FH * FW;
      }
      gemm(rx, g);
      r = o;
    }
    void* ro = ar.alloc(size_t(V) * FH * FW * OUT_HIDDEN * es);
    gemm(rx, conv_args(ray_out_conv_, dt_, r, V, FH, FW, 1, ro));
    if (out.ray_logits)
      pointwise_head(rx, dt_, PW_RAY, ro, long(V) * FH * FW, FH * FW, OUT_HIDDEN, 7, ray_out_w_, ray_out_b_,
                     out.ray_logits, nullptr, nullptr, nullptr, nullptr);

    void* fused = ar.alloc(size_t(V) * FH * FW * F * es);
    fusion_chain(depth_chain_, pyr, ph, pw, V, fused, ex, false);
    void* oc1 = ar.alloc(size_t(V) * FH * FW * (F / 2) * es);
    gemm(ex, conv_args(out_conv1_, dt_, fused, V, FH, FW, 1, oc1));
    void* up = ar.alloc(size_t(V) * H * W * (F / 2) * es);
    resize_bilinear(ex, dt_, oc1, V, FH, FW, F / 2, up, H, W, H, W, tb.uv_img, 0);
    void* o2 = ar.alloc(size_t(V) * H * W * OUT_HIDDEN * es);
    GemmArgs g = conv_args(oc2_0_, dt_, up, V, H, W, 1, o2);
    g.act = ACT_RELU;
    gemm(ex, g);
    pointwise_head(ex, dt_, PW_DEPTH, o2, long(V) * H * W, H * W, OUT_HIDDEN, 2, oc2_2_w_, oc2_2_b_, out.depth,
                   out.depth_conf, nullptr, nullptr, nullptr);
    ctx_.join(ex);
    ar.release(m);
  }

  // ---- camera head (depthanything3-rs/src/camera_head.rs:81-91)
  progress(SPLAT_STAGE_CAMERA_HEAD, 0);
  const int hin = 2 * d;
  float* h1 = ar.alloc_t<float>(size_t(V) * hin);
  float* h2 = ar.alloc_t<float>(size_t(V) * hin);
  small_linear(ex, cam_h_[0].dt, cam_tok, hin, V, hin, cam_h_[0].w, cam_h_[0].ldw, cam_h_[0].b, h1, hin, hin, ACT_RELU);
  small_linear(ex, cam_h_[1].dt, h1, hin, V, hin, cam_h_[1].w, cam_h_[1].ldw, cam_h_[1].b, h2, hin, hin, ACT_RELU);
  small_linear(ex, F32, h2, hin, V, hin, cam_t_.w, cam_t_.ldw, cam_t_.b, out.pose_encoding, 9, 3, ACT_NONE);
  small_linear(ex, F32, h2, hin, V, hin, cam_q_.w, cam_q_.ldw, cam_q_.b, out.pose_encoding + 3, 9, 4, ACT_NONE);
  small_linear(ex, F32, h2, hin, V, hin, cam_f_.w, cam_f_.ldw, cam_f_.b, out.pose_encoding + 7, 9, 2, ACT_RELU);
}

}  // namespace splat
