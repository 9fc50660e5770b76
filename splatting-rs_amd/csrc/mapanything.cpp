// MapAnything: weights (mapanything-rs/src/{model.rs:69-81, dinov2.rs:90-101,
// info_sharing.rs:39-47, dpt.rs:147-182,254-273, heads.rs:55-121, ray_encoder.rs:56-76}) and
// the forward of MapAnything::forward (model.rs:86-144), all views batched; views with known
// intrinsics add the ray encoder's features to their patches (model.rs:97-102).
#include <algorithm>
#include <cstring>

#include "runtime.h"

namespace splat {

namespace {
constexpr int PATCH = 14;
constexpr int KPATCH = 640;
constexpr float LN_EPS = 1e-6f;   // mapanything-rs/src/vit_block.rs:8
}  // namespace

MaModel::MaModel(Context& ctx, const SafeTensors& st, const splat_ma_spec& spec, int dt)
    : ctx_(ctx), spec_(spec), dt_(dt) {
  const int e = spec.enc_dim, d = spec.info_dim, F = spec.dpt_features;
  SPLAT_CHECK(e % 64 == 0 && d % 64 == 0 && e > 0 && d > 0, BAD_ARGUMENT, "MapAnything widths must be multiples of 64");
  SPLAT_CHECK(spec.enc_depth > 0 && spec.info_depth > 0, BAD_ARGUMENT, "MapAnything depths must be positive");
  SPLAT_CHECK(spec.hooks[0] < spec.hooks[1] && spec.hooks[1] < spec.hooks[2] && spec.hooks[2] == spec.info_depth - 1 &&
                  spec.hooks[0] >= 0,
              BAD_ARGUMENT, "MapAnything hooks must ascend to the last info block");
  SPLAT_CHECK(F % 16 == 0 && spec.pose_dim % 8 == 0 && spec.scale_dim > 0, BAD_ARGUMENT, "MapAnything head widths");
  for (int k = 0; k < 4; ++k) SPLAT_CHECK(spec.dpt_dims[k] % 8 == 0, BAD_ARGUMENT, "DPT widths must be multiples of 8");
  Loader L(ctx, st, dt, "");
  const std::string en = "encoder.model";
  {
    auto w = L.host(en + ".patch_embed.proj.weight", {e, 3, PATCH, PATCH});
    float* bias = L.vec(en + ".patch_embed.proj.bias", {e});
    patch_ = L.pack(w, e, 3 * PATCH * PATCH, bias, dt);
  }
  cls_ = L.vec(en + ".cls_token", {1, 1, e});
  pos_host_ = L.host(en + ".pos_embed", {1, 1 + 37 * 37, e});
  for (int i = 0; i < spec.enc_depth; ++i)
    enc_.push_back(L.block(en + ".blocks." + std::to_string(i), e, spec.enc_hidden, spec.enc_ffn == 1, false));
  fusion_norm_ = L.ln("fusion_norm_layer", e);
  scale_token_ = L.vec("scale_token", {d});
  has_proj_ = e != d;
  if (has_proj_) proj_embed_ = L.linear("info_sharing.proj_embed", d, e);
  for (int i = 0; i < spec.info_depth; ++i)
    info_.push_back(L.block("info_sharing.self_attention_blocks." + std::to_string(i), d, spec.info_hidden,
                            spec.info_ffn == 1, false));
  info_norm_ = L.ln("info_sharing.norm", d);
  view_pos_ = L.vec("info_sharing.view_pos_table", {1, d});
  const int* c = spec.dpt_dims;
  for (int h = 0; h < 4; ++h) {
    const std::string p = "dense_head.0.input_process." + std::to_string(h);
    dpt_proj_[h] = L.conv(p + ".0.0", c[h], h == 0 ? e : d, 1).lin;
    rn_[h] = L.conv(p + ".1", F, c[h], 3, false);
  }
  rs0_ = L.convt("dense_head.0.input_process.0.0.1", c[0], c[0], 4);
  rs1_ = L.convt("dense_head.0.input_process.1.0.1", c[1], c[1], 2);
  rs3_ = L.conv("dense_head.0.input_process.3.0.1", c[3], c[3], 3);
  for (int level = 1; level <= 4; ++level)
    chain_[level - 1] = load_fusion(L, "dense_head.0.scratch.refinenet" + std::to_string(level), F, level < 4);
  head1_ = L.conv("dense_head.1.conv1", F / 2, F, 3);
  head2_ = L.conv("dense_head.1.conv2.0", F / 2, F / 2, 3);
  head3_w_ = L.vec("dense_head.1.conv2.2.weight", {6, F / 2, 1, 1});
  head3_b_ = L.vec("dense_head.1.conv2.2.bias", {6});
  const int pd = spec.pose_dim;
  pose_proj_ = L.conv("pose_head.proj", pd, d, 1).lin;
  for (int blk = 0; blk < 2; ++blk)
    for (int k = 0; k < 3; ++k)
      pose_res_[blk][k] =
          L.conv("pose_head.res_conv." + std::to_string(blk) + ".res_conv" + std::to_string(k + 1), pd, pd, 1).lin;
  pose_mlp_[0] = L.linear("pose_head.more_mlps.0", pd, pd);
  pose_mlp_[1] = L.linear("pose_head.more_mlps.2", pd, pd);
  pose_t_ = L.linear("pose_head.fc_t", 3, pd);
  pose_rot_ = L.linear("pose_head.fc_rot", 4, pd);
  const int sd = spec.scale_dim;
  scale_proj_ = L.linear("scale_head.proj", sd, d);
  scale_mlp_[0] = L.linear("scale_head.mlp.0.0", sd, sd);
  scale_mlp_[1] = L.linear("scale_head.mlp.1.0", sd, sd);
  scale_out_ = L.linear("scale_head.output_proj", 1, sd);
  // The reference always builds the ray encoder (model.rs:73); a checkpoint without it still
  // serves unknown cameras here, and a forward with known ones reports the missing keys.
  has_rays_ = st.has("ray_dirs_encoder.conv_in.weight");
  if (has_rays_) {
    Loader LR(ctx, st, F32, "ray_dirs_encoder.");
    const int w[3] = {3 * PATCH * PATCH, 768, 1024};
    ray_in_ = LR.conv("conv_in", w[0], w[0], 3);
    for (int i = 0; i < 2; ++i) {
      const std::string b = "encoder." + std::to_string(i);
      ray_c1_[i] = LR.conv(b + ".conv1", w[i + 1], w[i], 3);
      ray_c2_[i] = LR.conv(b + ".conv2", w[i + 1], w[i + 1], 3);
      ray_sc_[i] = LR.conv(b + ".shortcut", w[i + 1], w[i], 1);
    }
    ray_out_ = LR.conv("encoder.2", e, w[2], 1);
    ray_norm_ = LR.ln("norm_layer", e);
  }
}

void MaModel::prepare(int V, int H, int W) {
  (void)V;
  const int R = H / PATCH, C = W / PATCH;
  auto key = std::make_tuple(R, C);
  if (tables_.count(key)) return;
  Tables t;
  auto pos = resize_pos_embed(pos_host_, spec_.enc_dim, R, C);
  t.pos = static_cast<float*>(ctx_.pool.upload(pos.data(), pos.size() * 4));
  tables_[key] = t;
}

void MaModel::forward(const float* images, int V, int H, int W, const splat_ma_out& out, float* enc_tokens,
                      bool encoder_only, const Hooks& hooks, const double* cam) {
  const Exec& ex = ctx_.ex;
  Arena& ar = ctx_.arena;
  const int R = H / PATCH, C = W / PATCH, P = R * C, n = P + 1;
  const int e = spec_.enc_dim, d = spec_.info_dim, F = spec_.dpt_features;
  const size_t es = dtype_size(dt_);
  const Tables& tb = tables_.at(std::make_tuple(R, C));
  std::vector<float> tap_host;
  auto tap = [&](int block, const float* x, long rows, int dim) {
    if (!hooks.tap || ex.dry) return;
    tap_host.resize(size_t(rows) * dim);
    SPLAT_HIP(hipMemcpyAsync(tap_host.data(), x, tap_host.size() * 4, hipMemcpyDeviceToHost, ex.stream));
    SPLAT_HIP(hipStreamSynchronize(ex.stream));
    hooks.tap(block, tap_host.data(), int(rows), dim, hooks.tap_user);
  };
  auto progress = [&](int stage, int block) {
    if (hooks.progress && !ex.dry) hooks.progress(stage, block, hooks.progress_user);
  };

  // ---- encoder (mapanything-rs/src/dinov2.rs:129-145), views batched: sequences of n tokens
  const long Te = long(V) * n;
  float* xe = enc_tokens ? enc_tokens : ar.alloc_t<float>(size_t(Te) * e);
  {
    const size_t m = ar.mark();
    void* patches = ar.alloc(size_t(V) * P * KPATCH * es);
    im2col_patch(ex, dt_, images, V, H, W, patches, KPATCH);
    GemmArgs g = lin_args(patch_, dt_, patches, KPATCH, V * P, xe, e);
    g.K = KPATCH;
    g.addtab = tb.pos + e;
    g.addtab_period = P;
    g.out_f32 = 1;
    g.rm_P = P;
    g.rm_n = n;
    g.rm_off = 1;
    gemm(ex, g);
    write_class_rows(ex, xe, V, n, e, cls_, tb.pos);
    ar.release(m);
  }
  {
    const size_t m = ar.mark();
    BlockScratch s;
    block_scratch(ctx_, s, dt_, Te, e, spec_.enc_hidden);
    for (int i = 0; i < spec_.enc_depth; ++i) {
      progress(SPLAT_STAGE_BLOCK, i);
      block_forward(ctx_, enc_[i], dt_, xe, xe, Te, V, n, s, 0, n, C, nullptr, 0, i);
      tap(i, xe, Te, e);
    }
    ar.release(m);
  }
  if (encoder_only) return;

  // ---- known cameras (model.rs:97-102): ray features added to the image patches, in fp32
  // (ray_encoder.rs:78-86: pixel-unshuffle, conv_in, two residual blocks
  // gelu(conv2(gelu(conv1(x))) + shortcut(x)), 1x1 to enc_dim, LayerNorm). Every view is
  // encoded; the add skips the views whose camera is unknown.
  if (cam) {
    SPLAT_CHECK(has_rays_, MISSING_KEY, "ray_dirs_encoder.* (known intrinsics need the ray encoder)");
    const size_t m = ar.mark();
    const long rows = long(V) * P;
    float* rays = ar.alloc_t<float>(size_t(rows) * 588);
    ray_unshuffled(ex, cam, V, H, W, rays);
    float* x = ar.alloc_t<float>(size_t(rows) * 588);
    gemm(ex, conv_args(ray_in_, F32, rays, V, R, C, 1, x));
    for (int i = 0; i < 2; ++i) {
      const int co = ray_c1_[i].cout;
      float* h = ar.alloc_t<float>(size_t(rows) * co);
      GemmArgs g1 = conv_args(ray_c1_[i], F32, x, V, R, C, 1, h);
      g1.act = ACT_GELU;
      gemm(ex, g1);
      float* sc = ar.alloc_t<float>(size_t(rows) * co);
      gemm(ex, conv_args(ray_sc_[i], F32, x, V, R, C, 1, sc));
      float* y = ar.alloc_t<float>(size_t(rows) * co);
      GemmArgs g2 = conv_args(ray_c2_[i], F32, h, V, R, C, 1, y);
      g2.res = sc;
      g2.ldres = co;
      g2.act_post = ACT_GELU;
      gemm(ex, g2);
      x = y;
    }
    float* f = ar.alloc_t<float>(size_t(rows) * e);
    gemm(ex, conv_args(ray_out_, F32, x, V, R, C, 1, f));
    float* fn = ar.alloc_t<float>(size_t(rows) * e);
    layer_norm(ex, F32, f, e, F32, fn, e, rows, e, ray_norm_.w, ray_norm_.b, LN_EPS);
    add_view_features(ex, xe, V, n, P, e, fn, cam);
    ar.release(m);
  }

  // ---- fusion norm on the patches (model.rs:106); the class token stays raw (model.rs:108)
  void* hook0 = ar.alloc(size_t(V) * P * e * es);
  layer_norm(ex, F32, xe, e, dt_, hook0, e, V * P, e, fusion_norm_.w, fusion_norm_.b, LN_EPS, P, n, 1);
  // ---- info-sharing sequence (info_sharing.rs:57-71): per view [patches, class], view 0 +
  // view_pos_table, the scale token last.
  const long Ti = long(V) * n + 1;
  float* xi = ar.alloc_t<float>(size_t(Ti) * d);
  if (has_proj_) {
    GemmArgs g = lin_args(proj_embed_, dt_, hook0, e, V * P, xi, d);
    g.out_f32 = 1;
    g.rm_P = P;
    g.rm_n = n;
    g.rm_off = 0;
    gemm(ex, g);
    const size_t m = ar.mark();
    void* cls_t = ar.alloc(size_t(V) * e * es);
    convert_rows(ex, F32, xe, long(n) * e, dt_, cls_t, e, V, e);  // the class token of each view
    GemmArgs gc = lin_args(proj_embed_, dt_, cls_t, e, V, xi, d);
    gc.out_f32 = 1;
    gc.rm_P = 1;
    gc.rm_n = n;
    gc.rm_off = P;
    gemm(ex, gc);
    ar.release(m);
  } else {
    // fp32 normed patches, then per view [patches, class]
    const size_t m = ar.mark();
    float* tmp = ar.alloc_t<float>(size_t(V) * P * d);
    layer_norm(ex, F32, xe, e, F32, tmp, d, V * P, e, fusion_norm_.w, fusion_norm_.b, LN_EPS, P, n, 1);
    for (int v = 0; v < V; ++v) copy_rows_f32(ex, xi + size_t(v) * n * d, d, tmp + size_t(v) * P * d, d, P, d);
    copy_rows_f32(ex, xi + size_t(P) * d, long(n) * d, xe, long(n) * e, V, d);
    ar.release(m);
  }
  add_rows(ex, xi, n, d, view_pos_);
  copy_rows_f32(ex, xi + size_t(V) * n * d, d, scale_token_, d, 1, d);

  // ---- alternating attention (info_sharing.rs:74-86): even blocks global over every token
  // (the scale token included), odd blocks per view (the scale token waits).
  void* hk[3];
  for (int k = 0; k < 3; ++k) hk[k] = ar.alloc(size_t(V) * P * d * es);
  float* scale_tok = ar.alloc_t<float>(d);
  {
    const size_t m = ar.mark();
    BlockScratch s;
    block_scratch(ctx_, s, dt_, Ti, d, spec_.info_hidden);
    int stored = 0;
    for (int i = 0; i < spec_.info_depth; ++i) {
      progress(SPLAT_STAGE_BLOCK, spec_.enc_depth + i);
      if (i % 2 == 0) block_forward(ctx_, info_[i], dt_, xi, xi, Ti, 1, int(Ti), s, 0, n, C, nullptr, 0, spec_.enc_depth + i);
      else block_forward(ctx_, info_[i], dt_, xi, xi, long(V) * n, V, n, s, 0, n, C, nullptr, 0, spec_.enc_depth + i);
      tap(spec_.enc_depth + i, xi, Ti, d);
      if (stored < 3 && i == spec_.hooks[stored]) {
        layer_norm(ex, F32, xi, d, dt_, hk[stored], d, V * P, d, info_norm_.w, info_norm_.b, LN_EPS, P, n, 0);
        if (stored == 2)
          layer_norm(ex, F32, xi + size_t(V) * n * d, d, F32, scale_tok, d, 1, d, info_norm_.w, info_norm_.b, LN_EPS);
        ++stored;
      }
    }
    ar.release(m);
  }

  // ---- scale head (heads.rs:122-129)
  progress(SPLAT_STAGE_DENSE_HEAD, 0);
  const int sd = spec_.scale_dim;
  float* scale = out.scale ? out.scale : ar.alloc_t<float>(1);
  {
    float* s1 = ar.alloc_t<float>(sd);
    float* s2 = ar.alloc_t<float>(sd);
    small_linear(ex, dt_, scale_tok, d, 1, d, scale_proj_.w, scale_proj_.ldw, scale_proj_.b, s1, sd, sd, ACT_NONE);
    small_linear(ex, dt_, s1, sd, 1, sd, scale_mlp_[0].w, scale_mlp_[0].ldw, scale_mlp_[0].b, s2, sd, sd, ACT_RELU);
    small_linear(ex, dt_, s2, sd, 1, sd, scale_mlp_[1].w, scale_mlp_[1].ldw, scale_mlp_[1].b, s1, sd, sd, ACT_RELU);
    small_linear(ex, dt_, s1, sd, 1, sd, scale_out_.w, scale_out_.ldw, scale_out_.b, scale, 1, 1, ACT_NONE);
    exp_clamp(ex, scale, 1, 1e-8f);
  }

  // ---- dense head (dpt.rs:277-302), views batched
  const int* c = spec_.dpt_dims;
  const int R2 = (R - 1) / 2 + 1, C2 = (C - 1) / 2 + 1;
  const int ph[4] = {4 * R, 2 * R, R, R2}, pw[4] = {4 * C, 2 * C, C, C2};
  const void* hooks_in[4] = {hook0, hk[0], hk[1], hk[2]};
  const int hook_dim[4] = {e, d, d, d};
  {
    const size_t mdpt = ar.mark();
    void* pyr[4];
    for (int k = 0; k < 4; ++k) pyr[k] = ar.alloc(size_t(V) * ph[k] * pw[k] * F * es);
    for (int k = 0; k < 4; ++k) {
      const size_t m = ar.mark();
      void* pk = ar.alloc(size_t(V) * P * c[k] * es);
      gemm(ex, lin_args(dpt_proj_[k], dt_, hooks_in[k], hook_dim[k], V * P, pk, c[k]));
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
        gemm(ex, u);
        r = up;
      } else if (k == 3) {
        void* dn = ar.alloc(size_t(V) * R2 * C2 * c[k] * es);
        gemm(ex, conv_args(rs3_, dt_, pk, V, R, C, 2, dn));
        r = dn;
      }
      gemm(ex, conv_args(rn_[k], dt_, r, V, ph[k], pw[k], 1, pyr[k]));
      ar.release(m);
    }
    // Coarsest first; each level upsamples 2x and is cropped to the next finer level
    // (dpt.rs:185-194); the finest is upsampled 2x uncropped.
    void* t3 = ar.alloc(size_t(V) * ph[2] * pw[2] * F * es);
    fusion_block(ctx_, dt_, chain_[3], pyr[3], nullptr, V, ph[3], pw[3], 2 * ph[3], 2 * pw[3], ph[2], pw[2], t3);
    void* t2 = ar.alloc(size_t(V) * ph[1] * pw[1] * F * es);
    fusion_block(ctx_, dt_, chain_[2], t3, pyr[2], V, ph[2], pw[2], 2 * ph[2], 2 * pw[2], ph[1], pw[1], t2);
    void* t1 = ar.alloc(size_t(V) * ph[0] * pw[0] * F * es);
    fusion_block(ctx_, dt_, chain_[1], t2, pyr[1], V, ph[1], pw[1], 2 * ph[1], 2 * pw[1], ph[0], pw[0], t1);
    const int FH = 2 * ph[0], FW = 2 * pw[0];
    void* path = ar.alloc(size_t(V) * FH * FW * F * es);
    fusion_block(ctx_, dt_, chain_[0], t1, pyr[0], V, ph[0], pw[0], FH, FW, FH, FW, path);
    void* h1 = ar.alloc(size_t(V) * FH * FW * (F / 2) * es);
    gemm(ex, conv_args(head1_, dt_, path, V, FH, FW, 1, h1));
    void* up = ar.alloc(size_t(V) * H * W * (F / 2) * es);
    resize_bilinear(ex, dt_, h1, V, FH, FW, F / 2, up, H, W, H, W, nullptr, 0);
    GemmArgs g = conv_args(head2_, dt_, up, V, H, W, 1, nullptr);
    g.act = ACT_RELU;
    if (dt_ != F32 && F / 2 == 128 && head2_.cin % 64 == 0) {
      // 1x1 head and dense_output in the convolution's epilogue: the 128-channel map at full
      // resolution (312 MB at C4) is never written
      g.out = up;  // not written
      g.hw3 = head3_w_;
      g.hb3 = head3_b_;
      g.hscale = scale;
      g.hhw = H * W;
      g.ho0 = out.raw;
      g.ho1 = out.points;
      g.ho2 = out.conf;
      g.ho3 = out.mask;
      gemm(ex, g);
    } else {
      void* h2 = ar.alloc(size_t(V) * H * W * (F / 2) * es);
      g.out = h2;
      gemm(ex, g);
      pointwise_head(ex, dt_, PW_MA, h2, long(V) * H * W, H * W, F / 2, 6, head3_w_, head3_b_, out.raw, out.points,
                     out.conf, out.mask, scale);
    }
    ar.release(mdpt);
  }

  // ---- pose head (heads.rs:80-99) on the last normed info features
  {
    const int pd = spec_.pose_dim;
    const size_t m = ar.mark();
    void* x = ar.alloc(size_t(V) * P * pd * es);
    void* r1 = ar.alloc(size_t(V) * P * pd * es);
    void* r2 = ar.alloc(size_t(V) * P * pd * es);
    gemm(ex, lin_args(pose_proj_, dt_, hk[2], d, V * P, x, pd));
    for (int blk = 0; blk < 2; ++blk) {
      GemmArgs a = lin_args(pose_res_[blk][0], dt_, x, pd, V * P, r1, pd);
      a.act = ACT_RELU;
      gemm(ex, a);
      GemmArgs b = lin_args(pose_res_[blk][1], dt_, r1, pd, V * P, r2, pd);
      b.act = ACT_RELU;
      gemm(ex, b);
      GemmArgs cc = lin_args(pose_res_[blk][2], dt_, r2, pd, V * P, x, pd);
      cc.act = ACT_RELU;
      cc.res = x;
      cc.ldres = pd;
      gemm(ex, cc);
    }
    float* pooled = ar.alloc_t<float>(size_t(V) * pd);
    float* m1 = ar.alloc_t<float>(size_t(V) * pd);
    mean_rows(ex, dt_, x, V, P, pd, pooled);
    small_linear(ex, dt_, pooled, pd, V, pd, pose_mlp_[0].w, pose_mlp_[0].ldw, pose_mlp_[0].b, m1, pd, pd, ACT_RELU);
    small_linear(ex, dt_, m1, pd, V, pd, pose_mlp_[1].w, pose_mlp_[1].ldw, pose_mlp_[1].b, pooled, pd, pd, ACT_RELU);
    float* quat = out.quaternion ? out.quaternion : ar.alloc_t<float>(size_t(V) * 4);
    small_linear(ex, dt_, pooled, pd, V, pd, pose_rot_.w, pose_rot_.ldw, pose_rot_.b, quat, 4, 4, ACT_NONE);
    normalize_rows(ex, quat, V, 4, 1e-8f);
    if (out.translation) {
      float* tr = ar.alloc_t<float>(size_t(V) * 3);
      small_linear(ex, dt_, pooled, pd, V, pd, pose_t_.w, pose_t_.ldw, pose_t_.b, tr, 3, 3, ACT_NONE);
      scale_rows(ex, tr, V, 3, scale, out.translation);
    }
    ar.release(m);
  }
}

}  // namespace splat
