// Host runtime: device context, activation arena, weight containers and loaders, and the
// two models' forward orchestration (da3.cpp, mapanything.cpp).
#pragma once

#include <map>
#include <memory>
#include <string>
#include <tuple>
#include <vector>

#include "../../include/splathip.h"
#include "host_tables.h"
#include "kernels.h"
#include "safetensors.h"

namespace splat {

// --- device memory --------------------------------------------------------------------------

// Weight and table allocations live until the context is destroyed.
class DevicePool {
 public:
  ~DevicePool();
  void* alloc(size_t bytes);
  void* upload(const void* host, size_t bytes);
  size_t bytes() const { return total_; }

 private:
  std::vector<void*> ptrs_;
  size_t total_ = 0;
};

// Bump allocator over one device allocation, reset at the start of every forward. In dry
// mode it hands out addresses from a fake base and only records the high-water mark.
class Arena {
 public:
  ~Arena();
  void begin(bool dry);
  void* alloc(size_t bytes);
  size_t mark() const { return used_; }
  void release(size_t mark) { used_ = mark; }  // frees everything allocated after `mark`
  template <typename T> T* alloc_t(size_t count) { return static_cast<T*>(alloc(count * sizeof(T))); }
  size_t peak() const { return peak_; }
  bool reserve(size_t bytes);  // grows the real allocation (synchronises the device first); true if moved

 private:
  char* base_ = nullptr;
  size_t cap_ = 0, used_ = 0, peak_ = 0;
  bool dry_ = false;
};

// --- weights -------------------------------------------------------------------------------

// GEMM weight [N, ldw] (model dtype unless noted), K = logical reduction length.
struct Lin {
  void* w = nullptr;
  long ldw = 0;
  int N = 0, K = 0, dt = BF16;
  float* b = nullptr;
  float* c1 = nullptr;  // folded LayerNorm (Loader::linear_ln): sum_k w[n, k] of the stored weights
};
// Implicit-GEMM convolution weight [cout, ks*ks*cin] (k = (ky*ks + kx)*cin + ci).
struct Conv {
  Lin lin;
  int cout = 0, cin = 0, ks = 1;
};
// Transposed convolution with kernel == stride s: weight [(dy*s+dx)*cout + co, cin].
struct ConvT {
  Lin lin;
  int cin = 0, cout = 0, s = 1;
};
struct LN {
  float* w = nullptr;
  float* b = nullptr;
  int n = 0;
};
// A pre-norm block. norm1 is folded into qkv and norm2 into fc1 (Loader::linear_ln): they
// consume the un-normalised residual rows and their statistics (GemmArgs::ln_in).
struct Block {
  int dim = 0, heads = 0, hidden = 0;
  bool swiglu = false, qk = false;
  LN qn, kn;
  Lin qkv, proj, fc1, fc2;  // SwiGLU: fc1 = w12 (2*hidden outputs), fc2 = w3
  float* ls1 = nullptr;
  float* ls2 = nullptr;
};

class Context;

class Loader {
 public:
  Loader(Context& ctx, const SafeTensors& st, int dt, std::string prefix) : ctx_(ctx), st_(st), dt_(dt), pre_(std::move(prefix)) {}
  Lin linear(const std::string& name, int n_out, int n_in, bool bias = true, int dt = -1);
  Conv conv(const std::string& name, int cout, int cin, int ks, bool bias = true);
  ConvT convt(const std::string& name, int cin, int cout, int s);
  LN ln(const std::string& name, int n);
  float* vec(const std::string& name, const std::vector<int64_t>& shape);
  std::vector<float> host(const std::string& name, const std::vector<int64_t>& shape);
  Block block(const std::string& name, int dim, int hidden, bool swiglu, bool qk);
  // linear(LN(x)) with the LayerNorm `ln` (weight g, bias beta) folded in: weights w * g
  // (along K), bias b + w beta, c1 = row sums of the stored (rounded) folded weights. glu: a
  // SwiGLU w12 whose rows are stored interleaved for the fused gate (GemmArgs::glu).
  Lin linear_ln(const std::string& name, int n_out, int n_in, const std::string& ln, bool glu = false);
  int dt() const { return dt_; }
  // Uploads row-major [n, k] host weights padded to a multiple of 64 columns, as `dt`.
  Lin pack(std::vector<float>& rows, int n, int k, float* bias, int dt);

 private:
  Context& ctx_;
  const SafeTensors& st_;
  int dt_;
  std::string pre_;
};

// --- per-forward state -----------------------------------------------------------------------

struct Hooks {
  splat_progress_fn progress = nullptr;
  void* progress_user = nullptr;
  splat_tap_fn tap = nullptr;
  void* tap_user = nullptr;
  splat_branch_tap_fn branch_tap = nullptr;
  void* branch_user = nullptr;
  bool any() const { return progress || tap || branch_tap; }
};

// Scratch buffers of one transformer stack, sized for its largest block.
// The LayerNorms folded into qkv / fc1 read `lnst`, the row statistics of `ln_src` (groups of
// `ln_group` columns), and in bf16 mode `h`, its rows in bf16 (fp32 mode reads the residual
// rows themselves). block_forward refreshes them when `in` is another buffer; a caller that
// rewrites rows of ln_src in place must refresh those rows.
struct BlockScratch {
  void* h = nullptr;     // [rows, dim] residual rows in bf16 (bf16 mode)
  float* lnst = nullptr; // [rows, dim / ln_group, 2] (sum, sum of squares)
  int ln_group = 64;
  const float* ln_src = nullptr;
  void* qkv = nullptr;   // [rows, 3*dim]
  void* att = nullptr;   // [rows, dim]
  void* mid = nullptr;   // [rows, hidden] (SwiGLU: the gated product)
};

class Context;

void block_scratch(Context& ctx, BlockScratch& s, int dt, long rows, int dim, int hidden);
// One pre-norm transformer block over `rows` rows of `in` (fp32 [rows, dim]) into `out`
// (may equal `in`): sequences of L rows each (`seqs` of them); rope: 0 none, 1 within view,
// 2 across views (positions from n tokens per view and `cols` patch columns). `block` numbers
// the block for the context's branch taps.
void block_forward(Context& ctx, const Block& b, int dt, const float* in, float* out, long rows, int seqs, int L,
                   BlockScratch& s, int rope, int n, int cols, const float* rope_table, int npos, int block);
// Recomputes the row statistics (and the bf16 copy) of `rows` rows of x (row r at
// (r / rm_P) * rm_n + rm_off + r % rm_P when rm_P > 0) and makes x the scratch's ln_src.
void block_ln_refresh(Context& ctx, int dt, const float* x, int rows, int dim, BlockScratch& s, int rm_P = 0,
                      int rm_n = 0, int rm_off = 0);

// --- image preprocessing (preprocess.cpp) -----------------------------------------------------

// (resize_taps and the size rules: host_tables.h)
// Device RGBA8 [h, w, 4] -> device RGBA8 [nh, nw, 4] (synchronises the context's stream).
void resize_device(Context& c, const uint8_t* src, int w, int h, uint8_t* dst, int nw, int nh, int filter);
// mapanything-rs/src/image_input.rs:195-216 on a device RGBA8 batch [V, H, W, 4]: the normalised
// images and foreground, and the reference's error when a view has no foreground pixel
// (synchronises the context's stream).
void model_input(Context& c, const uint8_t* rgba, int V, int H, int W, float* images, uint8_t* foreground);
// The crates' preprocessing of decoded host RGBA8 images into the device model input.
void da3_model_inputs(Context& c, int n, const uint8_t* const* rgba, const int* widths, const int* heights, float* images,
                      uint8_t* foreground, int& H, int& W);
void ma_model_inputs(Context& c, int n, const uint8_t* const* rgba, const int* widths, const int* heights, float* images,
                     uint8_t* foreground, int& H, int& W);

// GEMM arguments of a convolution on an NHWC map [V, Hi, Wi, cin]: ks == 1 -> plain rows,
// ks == 3 -> implicit im2col with padding 1. The caller adds epilogue fields.
GemmArgs conv_args(const Conv& c, int dt, const void* in, int V, int Hi, int Wi, int stride, void* out);
// 1x1 projection / linear over `rows` rows.
GemmArgs lin_args(const Lin& l, int dt, const void* in, long lda, int rows, void* out, long ldc);

// DPT fusion block (depthanything3-rs/src/dpt.rs:130-137, mapanything-rs/src/dpt.rs:235-242):
// out_conv(resize(RCU2(x + RCU1(skip)))) with RCU(x) = conv2(relu(conv1(relu(x)))) + x; the
// resize samples an (oh_full, ow_full) grid and keeps its first (oh, ow). Computed as
// resize(out_conv(...)): the 1x1 conv commutes with a bilinear resize.
struct RcuW { Conv c1, c2; };
struct FusionW { bool skip = false; RcuW u1, u2; Lin out; };
// Launches on `on` (default: the context's stream). With keep_scratch its arena scratch stays
// allocated: a block on a second stream must not hand memory back while later allocations for
// the first stream may still overlap its kernels.
void fusion_block(Context& ctx, int dt, const FusionW& f, const void* x, const void* skip, int V, int h, int w,
                  int oh_full, int ow_full, int oh, int ow, void* out, const Exec* on = nullptr,
                  bool keep_scratch = false);
FusionW load_fusion(Loader& L, const std::string& prefix, int features, bool skip);

// --- models ----------------------------------------------------------------------------------

struct Da3Spec {
  int dim, heads, depth, swiglu, alt_start;
  int out_layers[4];
  int head_features;
  int stage_dims[4];
  int hidden() const;
};
Da3Spec da3_variant_spec(int variant);

class Da3Model {
 public:
  Da3Model(Context& ctx, const SafeTensors& st, int variant, int dt, int strategy);
  // images fp32 device [V,3,H,W]; out fields device pointers (nullable optional ones).
  void forward(const float* images, int V, int H, int W, const splat_da3_out& out, int32_t* ref_dev, const Hooks& hooks);
  void prepare(int V, int H, int W);  // per-grid host tables (outside any capture)
  int dim() const { return spec_.dim; }
  int dt() const { return dt_; }

 private:
  struct Tables {
    float* pos = nullptr;   // [1 + P, d] resized positional embedding
    float* rope = nullptr;  // [2][npos][16]
    int npos = 0;
    float* uv[4] = {};      // [P, stage_dim] per hook
    float* uv_img = nullptr;   // [H*W, F/2]
    float* uv_ray = nullptr;   // [64*P, F/2]
  };
  void fusion_chain(const FusionW* chain, void* const pyr[4], const int ph[4], const int pw[4], int V, void* out,
                    const Exec& ex, bool keep_scratch);

  Context& ctx_;
  Da3Spec spec_;
  int dt_, strategy_;
  Lin patch_;
  float* cls_ = nullptr;
  float* camera_ = nullptr;
  std::vector<float> pos_host_;
  LN norm_;
  std::vector<Block> blocks_;
  LN head_norm_;
  Lin proj_[4];
  ConvT rs0_, rs1_;
  Conv rs3_;
  Conv rn_[4];
  FusionW depth_chain_[4], ray_chain_[4];
  Conv out_conv1_, oc2_0_;
  float* oc2_2_w_ = nullptr;
  float* oc2_2_b_ = nullptr;
  Conv ray_pre_[5];
  Conv ray_out_conv_;
  float* ray_out_w_ = nullptr;
  float* ray_out_b_ = nullptr;
  Lin cam_h_[2], cam_t_, cam_q_, cam_f_;
  std::map<std::tuple<int, int>, Tables> tables_;
};

class MaModel {
 public:
  MaModel(Context& ctx, const SafeTensors& st, const splat_ma_spec& spec, int dt);
  // cam: NULL (no view has a known camera) or device f64 [V, 5] = fx, fy, cx, cy, known.
  void forward(const float* images, int V, int H, int W, const splat_ma_out& out, float* enc_tokens, bool encoder_only,
               const Hooks& hooks, const double* cam = nullptr);
  void prepare(int V, int H, int W);
  const splat_ma_spec& spec() const { return spec_; }
  bool has_ray_encoder() const { return has_rays_; }
  int dt() const { return dt_; }

 private:
  struct Tables { float* pos = nullptr; };

  Context& ctx_;
  splat_ma_spec spec_;
  int dt_;
  Lin patch_;
  float* cls_ = nullptr;
  std::vector<float> pos_host_;
  std::vector<Block> enc_, info_;
  LN fusion_norm_, info_norm_;
  float* scale_token_ = nullptr;
  float* view_pos_ = nullptr;
  Lin proj_embed_;
  bool has_proj_ = false;
  Lin dpt_proj_[4];
  ConvT rs0_, rs1_;
  Conv rs3_;
  Conv rn_[4];
  FusionW chain_[4];
  Conv head1_, head2_;
  float* head3_w_ = nullptr;
  float* head3_b_ = nullptr;
  Lin pose_proj_;
  Lin pose_res_[2][3];
  Lin pose_mlp_[2], pose_t_, pose_rot_;
  Lin scale_proj_, scale_mlp_[2], scale_out_;
  // known-camera ray encoder (ray_encoder.rs:56-76), fp32 whatever the model dtype
  bool has_rays_ = false;
  Conv ray_in_, ray_c1_[2], ray_c2_[2], ray_sc_[2], ray_out_;
  LN ray_norm_;
  std::map<std::tuple<int, int>, Tables> tables_;
};

// --- context ---------------------------------------------------------------------------------

class Context {
 public:
  explicit Context(int device);
  ~Context();

  int device = 0;
  hipStream_t stream = nullptr;
  Exec ex;
  DevicePool pool;
  Arena arena;
  Workspace ws;
  // A second stream (default priority) for an independent branch of a forward, with its own
  // split-K workspace. fork() makes it wait for everything enqueued on ex's stream so far and
  // returns the Exec to launch the branch with; join() makes ex's stream wait for the branch.
  // Both are event records / waits, so a captured forward captures the branch too.
  hipStream_t aux = nullptr;
  Workspace ws2;
  // This device's statically allocated attention scratch (attention_scratch), looked up at
  // creation: the allocation-free attention entry point's partials.
  void* attn_scratch = nullptr;
  hipEvent_t ev_fork = nullptr, ev_join = nullptr;
  Exec fork(const Exec& on);
  void join(const Exec& on);
  // Grows `ws` and `ws2` to their need (synchronises the streams first; the old buffers may be
  // in use). True if a buffer moved, which invalidates captured graphs.
  bool reserve_workspace();
  std::string last_error;
  bool graphs = false;
  Hooks hooks;
  std::unique_ptr<Profiler> profiler;

  std::unique_ptr<Da3Model> da3;
  std::unique_ptr<MaModel> ma;

  // Grow-only device buffers the host-pointer entry points stage inputs/outputs in.
  std::map<int, std::pair<void*, size_t>> staging;
  void* staging_buffer(int slot, size_t bytes);

  // Graph cache: key -> instantiated graph.
  struct GraphKey {
    int model, V, H, W;
    const void* in;
    std::vector<const void*> outs;
    bool operator<(const GraphKey& o) const {
      return std::tie(model, V, H, W, in, outs) < std::tie(o.model, o.V, o.H, o.W, o.in, o.outs);
    }
  };
  std::map<GraphKey, hipGraphExec_t> graph_cache;
  void clear_graphs();

  // Runs `body` once dry to size the arena, then for real (optionally captured / replayed
  // as a graph under `key`).
  template <typename F> void run(const GraphKey& key, bool use_graph, F&& body);
};

template <typename F>
void Context::run(const GraphKey& key, bool use_graph, F&& body) {
  if (use_graph) {
    auto it = graph_cache.find(key);
    if (it != graph_cache.end()) {
      SPLAT_HIP(hipGraphLaunch(it->second, stream));
      return;
    }
  }
  ex.dry = true;
  arena.begin(true);
  body();
  ex.dry = false;
  if (arena.reserve(arena.peak())) clear_graphs();
  if (reserve_workspace()) clear_graphs();
  arena.begin(false);
  if (!use_graph) {
    body();
    return;
  }
  hipGraph_t graph = nullptr;
  SPLAT_HIP(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal));
  try {
    body();
  } catch (...) {
    hipGraph_t g2 = nullptr;
    (void)hipStreamEndCapture(stream, &g2);
    if (g2) (void)hipGraphDestroy(g2);
    throw;
  }
  SPLAT_HIP(hipStreamEndCapture(stream, &graph));
  hipGraphExec_t exec = nullptr;
  hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);
  SPLAT_HIP(e);
  graph_cache[key] = exec;
  SPLAT_HIP(hipGraphLaunch(exec, stream));
}

}  // namespace splat
