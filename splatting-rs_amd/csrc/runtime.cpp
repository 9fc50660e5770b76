#include "runtime.h"

#include <array>
#include <cmath>
#include <functional>
#include <cstring>
#include <thread>

namespace splat {

// --- device memory --------------------------------------------------------------------------

DevicePool::~DevicePool() {
  for (void* p : ptrs_) (void)hipFree(p);
}

void* DevicePool::alloc(size_t bytes) {
  void* p = nullptr;
  SPLAT_HIP(hipMalloc(&p, bytes ? bytes : 16));
  ptrs_.push_back(p);
  total_ += bytes;
  return p;
}

void* DevicePool::upload(const void* host, size_t bytes) {
  void* p = alloc(bytes);
  SPLAT_HIP(hipMemcpy(p, host, bytes, hipMemcpyHostToDevice));
  return p;
}

Arena::~Arena() {
  if (base_) (void)hipFree(base_);
}

void Arena::begin(bool dry) {
  dry_ = dry;
  used_ = 0;
  if (dry) peak_ = 0;
}

void* Arena::alloc(size_t bytes) {
  const size_t off = used_;
  used_ += (bytes + 255) & ~size_t(255);
  if (dry_) {
    peak_ = std::max(peak_, used_);
    return reinterpret_cast<void*>(uintptr_t(0x100000) + off);
  }
  SPLAT_CHECK(used_ <= cap_, HIP_ERROR, "activation arena overflow");
  return base_ + off;
}

bool Arena::reserve(size_t bytes) {
  if (bytes <= cap_) return false;
  SPLAT_HIP(hipDeviceSynchronize());
  if (base_) SPLAT_HIP(hipFree(base_));
  base_ = nullptr;
  cap_ = 0;
  const size_t want = bytes + bytes / 8;
  SPLAT_HIP(hipMalloc(reinterpret_cast<void**>(&base_), want));
  cap_ = want;
  return true;
}

// --- weights -------------------------------------------------------------------------------

namespace {

void parallel_for(size_t n, const std::function<void(size_t, size_t)>& fn) {
  const size_t threads = n > (1u << 20) ? std::min<size_t>(16, std::max(1u, std::thread::hardware_concurrency())) : 1;
  if (threads <= 1) {
    fn(0, n);
    return;
  }
  std::vector<std::thread> pool;
  const size_t chunk = (n + threads - 1) / threads;
  for (size_t t = 0; t < threads; ++t) {
    const size_t a = t * chunk, b = std::min(n, a + chunk);
    if (a < b) pool.emplace_back(fn, a, b);
  }
  for (auto& th : pool) th.join();
}

}  // namespace

Lin Loader::pack(std::vector<float>& rows, int n, int k, float* bias, int dt) {
  Lin l;
  l.N = n;
  l.K = k;
  l.dt = dt;
  l.ldw = ((k + 63) / 64) * 64;
  l.b = bias;
  const size_t total = size_t(n) * l.ldw;
  if (dt == F32) {
    std::vector<float> buf(total, 0.f);
    parallel_for(size_t(n), [&](size_t a, size_t b) {
      for (size_t r = a; r < b; ++r) std::memcpy(&buf[r * l.ldw], &rows[r * k], sizeof(float) * k);
    });
    l.w = ctx_.pool.upload(buf.data(), total * 4);
  } else {  // bf16 or f16, rounded to nearest even
    std::vector<uint16_t> buf(total, 0);
    const bool half = dt == F16;
    parallel_for(size_t(n), [&](size_t a, size_t b) {
      for (size_t r = a; r < b; ++r)
        for (int c = 0; c < k; ++c) {
          const float v = rows[r * size_t(k) + c];
          buf[r * l.ldw + c] = half ? f2h(v) : f2bf(v);
        }
    });
    l.w = ctx_.pool.upload(buf.data(), total * 2);
  }
  return l;
}

std::vector<float> Loader::host(const std::string& name, const std::vector<int64_t>& shape) {
  return st_.f32(pre_ + name, shape);
}

float* Loader::vec(const std::string& name, const std::vector<int64_t>& shape) {
  auto h = host(name, shape);
  return static_cast<float*>(ctx_.pool.upload(h.data(), h.size() * 4));
}

Lin Loader::linear(const std::string& name, int n_out, int n_in, bool bias, int dt) {
  auto w = host(name + ".weight", {n_out, n_in});
  float* b = bias ? vec(name + ".bias", {n_out}) : nullptr;
  return pack(w, n_out, n_in, b, dt < 0 ? dt_ : dt);
}

Conv Loader::conv(const std::string& name, int cout, int cin, int ks, bool bias) {
  auto w = host(name + ".weight", {cout, cin, ks, ks});
  std::vector<float> r(w.size());
  const int kk = ks * ks;
  for (int o = 0; o < cout; ++o)
    for (int c = 0; c < cin; ++c)
      for (int t = 0; t < kk; ++t) r[(size_t(o) * kk + t) * cin + c] = w[(size_t(o) * cin + c) * kk + t];
  Conv cv;
  cv.cout = cout;
  cv.cin = cin;
  cv.ks = ks;
  float* b = bias ? vec(name + ".bias", {cout}) : nullptr;
  cv.lin = pack(r, cout, kk * cin, b, dt_);
  return cv;
}

ConvT Loader::convt(const std::string& name, int cin, int cout, int s) {
  auto w = host(name + ".weight", {cin, cout, s, s});
  auto b = host(name + ".bias", {cout});
  const int n = s * s * cout;
  std::vector<float> r(size_t(n) * cin);
  std::vector<float> bx(n);
  for (int ci = 0; ci < cin; ++ci)
    for (int co = 0; co < cout; ++co)
      for (int t = 0; t < s * s; ++t) r[(size_t(t) * cout + co) * cin + ci] = w[(size_t(ci) * cout + co) * s * s + t];
  for (int t = 0; t < s * s; ++t)
    for (int co = 0; co < cout; ++co) bx[size_t(t) * cout + co] = b[co];
  ConvT ct;
  ct.cin = cin;
  ct.cout = cout;
  ct.s = s;
  float* bd = static_cast<float*>(ctx_.pool.upload(bx.data(), bx.size() * 4));
  ct.lin = pack(r, n, cin, bd, dt_);
  return ct;
}

Lin Loader::linear_ln(const std::string& name, int n_out, int n_in, const std::string& ln, bool glu) {
  auto w = host(name + ".weight", {n_out, n_in});
  auto b = host(name + ".bias", {n_out});
  if (glu) {  // rows 16j + i: x1 row 8j + i (i < 8), then x2 row hidden + 8j + i - 8
    const int hidden = n_out / 2;
    SPLAT_CHECK(n_out % 16 == 0, SHAPE_MISMATCH, name + ": SwiGLU hidden width must be a multiple of 8");
    std::vector<float> w2(w.size()), b2(b.size());
    for (int r = 0; r < n_out; ++r) {
      const int j = r / 16, i = r % 16, src = i < 8 ? 8 * j + i : hidden + 8 * j + i - 8;
      std::memcpy(&w2[size_t(r) * n_in], &w[size_t(src) * n_in], sizeof(float) * n_in);
      b2[r] = b[src];
    }
    w.swap(w2);
    b.swap(b2);
  }
  const auto g = host(ln + ".weight", {n_in});
  const auto beta = host(ln + ".bias", {n_in});
  std::vector<float> c2(n_out);
  std::vector<float> c1(n_out);
  parallel_for(size_t(n_out), [&](size_t a, size_t e) {
    for (size_t r = a; r < e; ++r) {
      double sb = b[r], s1 = 0.0;
      float* row = &w[r * size_t(n_in)];
      for (int k = 0; k < n_in; ++k) {
        sb += double(beta[k]) * row[k];
        row[k] *= g[k];
        // the stored value
        s1 += dt_ == F32 ? double(row[k]) : dt_ == F16 ? double(h2f(f2h(row[k]))) : double(bf2f(f2bf(row[k])));
      }
      c2[r] = float(sb);
      c1[r] = float(s1);
    }
  });
  float* bias = static_cast<float*>(ctx_.pool.upload(c2.data(), c2.size() * 4));
  Lin l = pack(w, n_out, n_in, bias, dt_);
  l.c1 = static_cast<float*>(ctx_.pool.upload(c1.data(), c1.size() * 4));
  return l;
}

LN Loader::ln(const std::string& name, int n) {
  LN l;
  l.n = n;
  l.w = vec(name + ".weight", {n});
  l.b = vec(name + ".bias", {n});
  return l;
}

Block Loader::block(const std::string& p, int dim, int hidden, bool swiglu, bool qk) {
  Block b;
  b.dim = dim;
  b.heads = dim / 64;
  b.hidden = hidden;
  b.swiglu = swiglu;
  b.qk = qk;
  b.qkv = linear_ln(p + ".attn.qkv", 3 * dim, dim, p + ".norm1");
  if (qk) {
    b.qn = ln(p + ".attn.q_norm", 64);
    b.kn = ln(p + ".attn.k_norm", 64);
  }
  b.proj = linear(p + ".attn.proj", dim, dim);
  b.ls1 = vec(p + ".ls1.gamma", {dim});
  if (swiglu) {
    b.fc1 = linear_ln(p + ".mlp.w12", 2 * hidden, dim, p + ".norm2", true);
    b.fc2 = linear(p + ".mlp.w3", dim, hidden);
  } else {
    b.fc1 = linear_ln(p + ".mlp.fc1", hidden, dim, p + ".norm2");
    b.fc2 = linear(p + ".mlp.fc2", dim, hidden);
  }
  b.ls2 = vec(p + ".ls2.gamma", {dim});
  return b;
}

// --- transformer block ----------------------------------------------------------------------

void block_scratch(Context& ctx, BlockScratch& s, int dt, long rows, int dim, int hidden) {
  const size_t es = dtype_size(dt);
  SPLAT_CHECK(dim % 64 == 0, BAD_ARGUMENT, "transformer width must be a multiple of 64");
  s.h = dt == F32 ? nullptr : ctx.arena.alloc(rows * dim * es);
  s.ln_group = dim <= 1024 ? 64 : 128;  // at most 16 partials a row for the folded consumers
  SPLAT_CHECK(dim % s.ln_group == 0 && dim / s.ln_group <= 16, BAD_ARGUMENT, "transformer width for the folded norms");
  s.lnst = ctx.arena.alloc_t<float>(size_t(rows) * (dim / s.ln_group) * 2);
  s.ln_src = nullptr;
  s.qkv = ctx.arena.alloc(rows * 3 * dim * es);
  s.att = ctx.arena.alloc(rows * dim * es);
  s.mid = ctx.arena.alloc(rows * hidden * es);
}

void block_forward(Context& ctx, const Block& b, int dt, const float* in, float* out, long rows, int seqs, int L,
                   BlockScratch& s, int rope, int n, int cols, const float* rope_table, int npos, int block) {
  const Exec& ex = ctx.ex;
  const int d = b.dim;
  // Branch tap: the branch's last GEMM again, bias only (no LayerScale, no residual), into an
  // fp32 temporary that is copied to the host (the dry run sizes the temporary too).
  auto branch_tap = [&](int which, const Lin& l, const void* A, long lda, int K) {
    const Hooks& hk = ctx.hooks;
    if (!hk.branch_tap) return;
    const size_t m = ctx.arena.mark();
    float* y = ctx.arena.alloc_t<float>(size_t(rows) * d);
    GemmArgs g = lin_args(l, dt, A, lda, int(rows), y, d);
    g.K = K;
    g.out_f32 = 1;
    gemm(ex, g);
    if (!ex.dry) {
      std::vector<float> host(size_t(rows) * d);
      SPLAT_HIP(hipMemcpyAsync(host.data(), y, host.size() * 4, hipMemcpyDeviceToHost, ex.stream));
      SPLAT_HIP(hipStreamSynchronize(ex.stream));
      hk.branch_tap(block, which, host.data(), int(rows), d, hk.branch_user);
    }
    ctx.arena.release(m);
  };
  // The LayerNorms (eps 1e-6, vit_block.rs:15 / mapanything vit_block.rs:8) are folded into
  // qkv and fc1: they read the residual rows before the norm (bf16 copy or fp32) and the row
  // statistics that the previous residual epilogue wrote.
  if (s.ln_src != in) block_ln_refresh(ctx, dt, in, int(rows), d, s);
  const void* xin = dt == F32 ? static_cast<const void*>(in) : s.h;
  auto fold = [&](GemmArgs& a, const Lin& l) {
    a.ln_in = s.lnst;
    a.ln_parts = d / s.ln_group;
    a.ln_c1 = l.c1;
    a.ln_eps = 1e-6f;
  };
  auto emit = [&](GemmArgs& a) {  // residual epilogue: statistics (and bf16 copy) of its rows
    a.ln_out = s.lnst;
    a.ln_group = s.ln_group;
    a.ln_copy = dt == F32 ? nullptr : s.h;
  };
  // norm1 -> qkv
  GemmArgs g;
  g.dt = dt;
  g.M = int(rows);
  g.N = 3 * d;
  g.K = d;
  g.A = xin;
  g.lda = d;
  g.W = b.qkv.w;
  g.ldw = b.qkv.ldw;
  g.bias = b.qkv.b;
  g.out = s.qkv;
  g.ldc = 3 * d;
  fold(g, b.qkv);
  if (b.qk || rope) {  // qk-norm + RoPE in the epilogue (vit_block.rs:155-162)
    g.qk_dim = d;
    if (b.qk) {
      g.qw = b.qn.w;
      g.qb = b.qn.b;
      g.kw = b.kn.w;
      g.kb = b.kn.b;
    }
    if (rope) {
      g.rope_cs = rope_table;
      g.rope_n = n;
      g.rope_cols = cols;
      g.rope_across = rope == 2;
      g.rope_npos = npos;
    }
  }
  if (dt != F32) {  // Q leaves the epilogue times the softmax scale, rounded to bf16 or f16 once
    g.q_cols = d;
    g.q_scale = ATTN_Q_SCALE;
  }
  gemm(ex, g);
  // attention
  AttnArgs a;
  a.dt = dt;
  const size_t es = dtype_size(dt);
  a.q = s.qkv;
  a.k = static_cast<char*>(s.qkv) + d * es;
  a.v = static_cast<char*>(s.qkv) + 2 * d * es;
  a.ld = 3 * d;
  a.o = s.att;
  a.ldo = d;
  a.L = L;
  a.heads = b.heads;
  a.seqs = seqs;
  a.seq_stride = L;
  a.q_scaled = dt != F32;
  attention(ex, a);
  branch_tap(0, b.proj, s.att, d, d);
  // out = in + ls1 * proj(att)
  GemmArgs p;
  p.dt = dt;
  p.M = int(rows);
  p.N = d;
  p.K = d;
  p.A = s.att;
  p.lda = d;
  p.W = b.proj.w;
  p.ldw = b.proj.ldw;
  p.bias = b.proj.b;
  p.gamma = b.ls1;
  p.res = in;
  p.ldres = d;
  p.res_f32 = 1;
  p.out = out;
  p.ldc = d;
  p.out_f32 = 1;
  emit(p);
  gemm(ex, p);
  // out += ls2 * mlp(norm2(out))
  const void* xmid = dt == F32 ? static_cast<const void*>(out) : s.h;
  GemmArgs f1;
  f1.dt = dt;
  f1.M = int(rows);
  f1.K = d;
  f1.A = xmid;
  f1.lda = d;
  f1.W = b.fc1.w;
  f1.ldw = b.fc1.ldw;
  f1.bias = b.fc1.b;
  fold(f1, b.fc1);
  if (b.swiglu) {  // w3(silu(x1) * x2): the gate in the w12 epilogue (rows interleaved at load)
    f1.N = 2 * b.hidden;
    f1.glu = 1;
    f1.out = s.mid;
    f1.ldc = b.hidden;
    gemm(ex, f1);
  } else {
    f1.N = b.hidden;
    f1.act = ACT_GELU;
    f1.out = s.mid;
    f1.ldc = b.hidden;
    gemm(ex, f1);
  }
  branch_tap(1, b.fc2, s.mid, b.hidden, b.hidden);
  GemmArgs f2;
  f2.dt = dt;
  f2.M = int(rows);
  f2.N = d;
  f2.K = b.hidden;
  f2.A = s.mid;
  f2.lda = b.hidden;
  f2.W = b.fc2.w;
  f2.ldw = b.fc2.ldw;
  f2.bias = b.fc2.b;
  f2.gamma = b.ls2;
  f2.res = out;
  f2.ldres = d;
  f2.res_f32 = 1;
  f2.out = out;
  f2.ldc = d;
  f2.out_f32 = 1;
  emit(f2);
  gemm(ex, f2);
  s.ln_src = out;
}

void block_ln_refresh(Context& ctx, int dt, const float* x, int rows, int dim, BlockScratch& s, int rm_P, int rm_n,
                      int rm_off) {
  ln_stats(ctx.ex, x, dim, rows, dim, s.ln_group, s.lnst, dt, dt == F32 ? nullptr : s.h, rm_P, rm_n, rm_off);
  s.ln_src = x;
}

// --- DPT building blocks --------------------------------------------------------------------

GemmArgs lin_args(const Lin& l, int dt, const void* in, long lda, int rows, void* out, long ldc) {
  GemmArgs g;
  g.dt = dt;
  g.M = rows;
  g.N = l.N;
  g.K = l.K;
  g.A = in;
  g.lda = lda;
  g.W = l.w;
  g.ldw = l.ldw;
  g.bias = l.b;
  g.out = out;
  g.ldc = ldc;
  return g;
}

GemmArgs conv_args(const Conv& c, int dt, const void* in, int V, int Hi, int Wi, int stride, void* out) {
  if (c.ks == 1 && stride == 1) return lin_args(c.lin, dt, in, c.cin, V * Hi * Wi, out, c.cout);
  GemmArgs g = lin_args(c.lin, dt, in, 0, 0, out, c.cout);
  const int pad = c.ks / 2;
  g.amode = A_CONV;
  g.V = V;
  g.Hi = Hi;
  g.Wi = Wi;
  g.Cin = c.cin;
  g.ks = c.ks;
  g.stride = stride;
  g.pad = pad;
  g.Ho = (Hi + 2 * pad - c.ks) / stride + 1;
  g.Wo = (Wi + 2 * pad - c.ks) / stride + 1;
  g.M = V * g.Ho * g.Wo;
  return g;
}

void fusion_block(Context& ctx, int dt, const FusionW& f, const void* x, const void* skip, int V, int h, int w,
                  int oh_full, int ow_full, int oh, int ow, void* out, const Exec* on, bool keep_scratch) {
  const Exec& ex = on ? *on : ctx.ex;
  const int F = f.u2.c1.cin;
  const size_t bytes = size_t(V) * h * w * F * dtype_size(dt);
  const size_t mark = ctx.arena.mark();
  const void* xs = x;
  if (skip) {
    // xs = x + RCU1(skip) = x + skip + conv2(relu(conv1(relu(skip))))
    void* a = ctx.arena.alloc(bytes);
    GemmArgs g1 = conv_args(f.u1.c1, dt, skip, V, h, w, 1, a);
    g1.relu_in = 1;
    g1.act = ACT_RELU;
    gemm(ex, g1);
    void* xs2 = ctx.arena.alloc(bytes);
    GemmArgs g2 = conv_args(f.u1.c2, dt, a, V, h, w, 1, xs2);
    g2.res = skip;
    g2.ldres = F;
    g2.res2 = x;
    g2.ldres2 = F;
    gemm(ex, g2);
    xs = xs2;
  }
  void* a2 = ctx.arena.alloc(bytes);
  GemmArgs g3 = conv_args(f.u2.c1, dt, xs, V, h, w, 1, a2);
  g3.relu_in = 1;
  g3.act = ACT_RELU;
  gemm(ex, g3);
  void* y = ctx.arena.alloc(bytes);
  GemmArgs g4 = conv_args(f.u2.c2, dt, a2, V, h, w, 1, y);
  g4.res = xs;
  g4.ldres = F;
  gemm(ex, g4);
  // out_conv (1x1) before the bilinear resize instead of after: the resize's weights per output
  // pixel sum to 1, so the two commute exactly (bias included) and the 1x1 runs on a quarter
  // of the pixels
  void* z = ctx.arena.alloc(bytes);
  gemm(ex, lin_args(f.out, dt, y, F, V * h * w, z, F));
  resize_bilinear(ex, dt, z, V, h, w, F, out, oh_full, ow_full, oh, ow, nullptr, 0);
  if (!keep_scratch) ctx.arena.release(mark);
}

FusionW load_fusion(Loader& L, const std::string& p, int F, bool skip) {
  FusionW f;
  f.skip = skip;
  if (skip) {
    f.u1.c1 = L.conv(p + ".resConfUnit1.conv1", F, F, 3);
    f.u1.c2 = L.conv(p + ".resConfUnit1.conv2", F, F, 3);
  }
  f.u2.c1 = L.conv(p + ".resConfUnit2.conv1", F, F, 3);
  f.u2.c2 = L.conv(p + ".resConfUnit2.conv2", F, F, 3);
  f.out = L.conv(p + ".out_conv", F, F, 1).lin;
  return f;
}

// --- context ---------------------------------------------------------------------------------

Context::Context(int dev) : device(dev) {
  SPLAT_HIP(hipSetDevice(dev));
  attn_scratch = attention_scratch(dev);
  SPLAT_HIP(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
  SPLAT_HIP(hipStreamCreateWithFlags(&aux, hipStreamNonBlocking));
  SPLAT_HIP(hipEventCreateWithFlags(&ev_fork, hipEventDisableTiming));
  SPLAT_HIP(hipEventCreateWithFlags(&ev_join, hipEventDisableTiming));
  ex.stream = stream;
  ex.ws = &ws;
}

Exec Context::fork(const Exec& on) {
  Exec b = on;
  b.stream = aux;
  b.ws = &ws2;
  if (!on.dry) {
    SPLAT_HIP(hipEventRecord(ev_fork, on.stream));
    SPLAT_HIP(hipStreamWaitEvent(aux, ev_fork, 0));
  }
  return b;
}

void Context::join(const Exec& on) {
  if (on.dry) return;
  SPLAT_HIP(hipEventRecord(ev_join, aux));
  SPLAT_HIP(hipStreamWaitEvent(on.stream, ev_join, 0));
}

bool Context::reserve_workspace() {
  bool moved = false;
  for (Workspace* w : {&ws, &ws2}) {
    if (w->need <= w->cap) continue;
    SPLAT_HIP(hipStreamSynchronize(stream));
    SPLAT_HIP(hipStreamSynchronize(aux));
    if (w->ptr) SPLAT_HIP(hipFree(w->ptr));
    w->ptr = nullptr;
    w->cap = 0;
    SPLAT_HIP(hipMalloc(&w->ptr, w->need));
    w->cap = w->need;
    moved = true;
  }
  return moved;
}

Context::~Context() {
  (void)hipSetDevice(device);
  if (stream) (void)hipStreamSynchronize(stream);
  if (aux) (void)hipStreamSynchronize(aux);
  clear_graphs();
  da3.reset();
  ma.reset();
  for (auto& kv : staging)
    if (kv.second.first) (void)hipFree(kv.second.first);
  if (ws.ptr) (void)hipFree(ws.ptr);
  if (ws2.ptr) (void)hipFree(ws2.ptr);
  if (ev_fork) (void)hipEventDestroy(ev_fork);
  if (ev_join) (void)hipEventDestroy(ev_join);
  if (aux) (void)hipStreamDestroy(aux);
  if (stream) (void)hipStreamDestroy(stream);
}

void* Context::staging_buffer(int slot, size_t bytes) {
  auto& s = staging[slot];
  if (s.second < bytes) {
    SPLAT_HIP(hipStreamSynchronize(stream));
    if (s.first) SPLAT_HIP(hipFree(s.first));
    s.first = nullptr;
    s.second = 0;
    SPLAT_HIP(hipMalloc(&s.first, bytes));
    s.second = bytes;
  }
  return s.first;
}

void Context::clear_graphs() {
  for (auto& kv : graph_cache) (void)hipGraphExecDestroy(kv.second);
  graph_cache.clear();
}

}  // namespace splat
