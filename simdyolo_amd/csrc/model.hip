// C++ host mirror of the reference's model interpreter for the YOLOv8 detect
// family: parameter walk + BN fold (PtModel.cs:84-145), module semantics
// (PtModel.cs:267-317: Conv, C2f/Bottleneck, SPPF, Upsample, Concat) and the
// Detect head (PtModel.cs:444-504), planned for MI355X:
//
//  * every activation is an NHWC view; each Concat buffer is allocated first
//    and its inputs' producers write straight into their channel slices, and
//    C2f's chunk/concat are slices of one buffer, so no copies remain;
//  * the Bottleneck residual add is fused into the second conv's epilogue;
//  * Detect's first box and class convs share the level input and run as one
//    conv with concatenated output channels;
//  * a shape's op list is captured once into a hipGraph and replayed.
//
// Topology: ultralytics yolov8.yaml (the module tree the reference interprets).
#include <cmath>
#include <cstring>
#include <functional>
#include <map>
#include <tuple>

#include "sy_internal.h"

using namespace sy;

namespace {

struct ParamWalk {
  // enumeration output
  int32_t* layout = nullptr;
  int max_entries = 0;
  int count = 0;
  // consumption input
  const float* params = nullptr;
  size_t n_params = 0, pos = 0;
  bool overrun = false;

  const float* take(int kind, int d0, int d1, int d2, int d3, int fan_in) {
    if (layout && count < max_entries) {
      int32_t* e = layout + 6 * count;
      e[0] = kind; e[1] = d0; e[2] = d1; e[3] = d2; e[4] = d3; e[5] = fan_in;
    }
    ++count;
    const size_t len = (size_t)d0 * d1 * d2 * d3;
    const float* p = nullptr;
    if (params) {
      if (pos + len > n_params) overrun = true;
      else p = params + pos;
    }
    pos += len;
    return p;
  }
};

// Folded weights of one Conv (conv + BN + SiLU) or Conv2d (+ bias).
struct ConvW {
  int ic = 0, oc = 0, k = 1, s = 1;
  bool silu = true;
  std::vector<float> w, b;
};

ConvW read_conv(ParamWalk& pw, int ic, int oc, int k, int s, float eps) {
  ConvW c;
  c.ic = ic; c.oc = oc; c.k = k; c.s = s; c.silu = true;
  const float* w = pw.take(SY_P_CONV_WEIGHT, oc, ic, k, k, ic * k * k);
  const float* g = pw.take(SY_P_BN_GAMMA, oc, 1, 1, 1, 0);
  const float* be = pw.take(SY_P_BN_BETA, oc, 1, 1, 1, 0);
  const float* mu = pw.take(SY_P_BN_MEAN, oc, 1, 1, 1, 0);
  const float* va = pw.take(SY_P_BN_VAR, oc, 1, 1, 1, 0);
  if (w && g && be && mu && va) {
    c.w.resize((size_t)oc * ic * k * k);
    c.b.resize(oc);
    sy_fold_bn(w, oc, ic * k * k, nullptr, g, be, mu, va, eps, c.w.data(), c.b.data());
  }
  return c;
}

ConvW read_conv2d(ParamWalk& pw, int ic, int oc, int bias_kind) {
  ConvW c;
  c.ic = ic; c.oc = oc; c.k = 1; c.s = 1; c.silu = false;
  const float* w = pw.take(SY_P_CONV_WEIGHT, oc, ic, 1, 1, ic);
  const float* b = pw.take(bias_kind, oc, 1, 1, 1, 0);
  if (w && b) {
    c.w.assign(w, w + (size_t)oc * ic);
    c.b.assign(b, b + oc);
  }
  return c;
}

struct C2fW {
  ConvW cv1, cv2;
  std::vector<std::pair<ConvW, ConvW>> m;
  int c = 0;
  bool add = false;
};

C2fW read_c2f(ParamWalk& pw, int c1, int c2, int n, bool shortcut, float eps) {
  C2fW f;
  f.c = c2 / 2;
  f.add = shortcut;
  // state_dict order: cv1, cv2, m.0.cv1, m.0.cv2, ...
  f.cv1 = read_conv(pw, c1, 2 * f.c, 1, 1, eps);
  f.cv2 = read_conv(pw, (2 + n) * f.c, c2, 1, 1, eps);
  for (int i = 0; i < n; ++i) {
    ConvW a = read_conv(pw, f.c, f.c, 3, 1, eps);
    ConvW b = read_conv(pw, f.c, f.c, 3, 1, eps);
    f.m.emplace_back(std::move(a), std::move(b));
  }
  return f;
}

int scale_ch(const sy_model_config& c, int ch) {
  double v = (double)(ch < c.max_channels ? ch : c.max_channels) * c.width;
  return (int)(std::ceil(v / 8.0) * 8.0);
}
int scale_n(const sy_model_config& c, int n) {
  if (n <= 1) return n;
  int r = (int)std::lround((double)n * c.depth);
  return r < 1 ? 1 : r;
}

struct V8Weights {
  ConvW c0, c1, c3, c5, c7, c16, c19, s_cv1, s_cv2;
  C2fW f2, f4, f6, f8, f12, f15, f18, f21;
  ConvW box[3][3], cls[3][3];
  int ch[3] = {0, 0, 0}, box_ch = 0, cls_ch = 0;
};

void read_yolov8(ParamWalk& pw, const sy_model_config& cfg, V8Weights& m) {
  const float eps = cfg.bn_eps;
  const int c64 = scale_ch(cfg, 64), c128 = scale_ch(cfg, 128), c256 = scale_ch(cfg, 256), c512 = scale_ch(cfg, 512),
            c1024 = scale_ch(cfg, 1024);
  const int n3 = scale_n(cfg, 3), n6 = scale_n(cfg, 6);
  m.c0 = read_conv(pw, 3, c64, 3, 2, eps);
  m.c1 = read_conv(pw, c64, c128, 3, 2, eps);
  m.f2 = read_c2f(pw, c128, c128, n3, true, eps);
  m.c3 = read_conv(pw, c128, c256, 3, 2, eps);
  m.f4 = read_c2f(pw, c256, c256, n6, true, eps);
  m.c5 = read_conv(pw, c256, c512, 3, 2, eps);
  m.f6 = read_c2f(pw, c512, c512, n6, true, eps);
  m.c7 = read_conv(pw, c512, c1024, 3, 2, eps);
  m.f8 = read_c2f(pw, c1024, c1024, n3, true, eps);
  m.s_cv1 = read_conv(pw, c1024, c1024 / 2, 1, 1, eps);
  m.s_cv2 = read_conv(pw, c1024 / 2 * 4, c1024, 1, 1, eps);
  m.f12 = read_c2f(pw, c1024 + c512, c512, n3, false, eps);
  m.f15 = read_c2f(pw, c512 + c256, c256, n3, false, eps);
  m.c16 = read_conv(pw, c256, c256, 3, 2, eps);
  m.f18 = read_c2f(pw, c256 + c512, c512, n3, false, eps);
  m.c19 = read_conv(pw, c512, c512, 3, 2, eps);
  m.f21 = read_c2f(pw, c512 + c1024, c1024, n3, false, eps);
  m.ch[0] = c256; m.ch[1] = c512; m.ch[2] = c1024;
  int c2 = 16;
  if (c256 / 4 > c2) c2 = c256 / 4;
  if (4 * cfg.reg_max > c2) c2 = 4 * cfg.reg_max;
  int c3 = cfg.nc < 100 ? cfg.nc : 100;
  if (c256 > c3) c3 = c256;
  m.box_ch = c2;
  m.cls_ch = c3;
  for (int i = 0; i < 3; ++i) {
    m.box[i][0] = read_conv(pw, m.ch[i], c2, 3, 1, eps);
    m.box[i][1] = read_conv(pw, c2, c2, 3, 1, eps);
    m.box[i][2] = read_conv2d(pw, c2, 4 * cfg.reg_max, SY_P_BIAS_BOX);
  }
  for (int i = 0; i < 3; ++i) {
    m.cls[i][0] = read_conv(pw, m.ch[i], c3, 3, 1, eps);
    m.cls[i][1] = read_conv(pw, c3, c3, 3, 1, eps);
    m.cls[i][2] = read_conv2d(pw, c3, cfg.nc, SY_P_BIAS_CLS);
  }
}

int validate_cfg(const sy_model_config* cfg) {
  SY_CHECK(cfg, SY_EINVAL, "null model config");
  SY_CHECK(cfg->arch == SY_ARCH_YOLOV8, SY_EUNSUPPORTED, "unsupported architecture %d", cfg->arch);
  SY_CHECK(cfg->depth > 0 && cfg->width > 0 && cfg->max_channels > 0 && cfg->nc > 0 && cfg->reg_max > 0 &&
               cfg->bn_eps > 0,
           SY_EINVAL, "invalid model config");
  return SY_OK;
}

// ---------------------------------------------------------------- planning

struct Conv {
  uint64_t id = 0;
  int oc = 0;
};

struct Plan {
  int batch = 0, h = 0, w = 0;
  char* arena = nullptr;
  size_t bytes = 0;
  float* input = nullptr;   // [B,3,H,W] NCHW
  float* output = nullptr;  // [B,nc+4,A]
  std::vector<std::function<int()>> ops;
  uint64_t graph = 0;
  size_t scratch = 0;
};

}  // namespace

struct sy_model {
  sy_ctx* ctx = nullptr;
  sy_model_config cfg{};
  bool use_graph = true;
  size_t weight_bytes = 0;
  // prepared convs
  Conv c0, c1, c3, c5, c7, c16, c19, s_cv1, s_cv2;
  struct C2f {
    Conv cv1, cv2;
    std::vector<std::pair<Conv, Conv>> m;
    int c = 0;
    bool add = false;
  } f2, f4, f6, f8, f12, f15, f18, f21;
  Conv head0[3], box1[3], cls1[3], box2[3], cls2[3];
  int ch[3] = {0, 0, 0}, box_ch = 0, cls_ch = 0, c64 = 0, c128 = 0, c256 = 0, c512 = 0, c1024 = 0;
  std::map<std::tuple<int, int, int>, std::unique_ptr<Plan>> plans;
  ~sy_model() {
    if (!ctx) return;
    (void)hipStreamSynchronize(ctx->stream);
    for (auto& kv : plans) {
      if (kv.second->graph) sy_graph_destroy(ctx, kv.second->graph);
      if (kv.second->arena) (void)hipFree(kv.second->arena);
    }
  }
};

namespace {

int make_conv(sy_model* m, const ConvW& c, Conv* out) {
  const int p = c.k / 2;
  SY_TRY(sy_conv_create(m->ctx, c.w.data(), c.b.data(), c.oc, c.ic, c.k, c.k, c.s, c.s, p, p, p, p, 1, 1, 1,
                        c.silu ? 1 : 0, &out->id));
  out->oc = c.oc;
  m->weight_bytes += (c.w.size() + c.b.size()) * sizeof(float);
  return SY_OK;
}

int make_c2f(sy_model* m, const C2fW& f, sy_model::C2f* out) {
  SY_TRY(make_conv(m, f.cv1, &out->cv1));
  SY_TRY(make_conv(m, f.cv2, &out->cv2));
  out->m.resize(f.m.size());
  for (size_t i = 0; i < f.m.size(); ++i) {
    SY_TRY(make_conv(m, f.m[i].first, &out->m[i].first));
    SY_TRY(make_conv(m, f.m[i].second, &out->m[i].second));
  }
  out->c = f.c;
  out->add = f.add;
  return SY_OK;
}

struct Planner {
  sy_model* m;
  Plan* plan;
  size_t used = 0;
  std::vector<std::pair<sy_tensor*, size_t>> fixups;  // tensors whose data is an arena offset
  std::vector<std::unique_ptr<sy_tensor>> store;

  // Tensors are recorded with arena offsets and patched once the arena exists.
  sy_tensor* alloc(int n, int c, int h, int w) {
    used = (used + 255) & ~size_t(255);
    auto t = std::make_unique<sy_tensor>(sy_tensor{nullptr, n, c, h, w, c, SY_LAYOUT_NHWC});
    fixups.emplace_back(t.get(), used);
    used += (size_t)n * c * h * w * sizeof(float);
    store.push_back(std::move(t));
    return store.back().get();
  }
  // Channel slice view; resolved after the parent.
  sy_tensor* slice(sy_tensor* parent, int c0, int cn) {
    auto t = std::make_unique<sy_tensor>(*parent);
    t->c = cn;
    slices.emplace_back(t.get(), parent, c0);
    store.push_back(std::move(t));
    return store.back().get();
  }
  std::vector<std::tuple<sy_tensor*, sy_tensor*, int>> slices;

  void conv(const Conv& c, sy_tensor* x, sy_tensor* y, sy_tensor* res = nullptr) {
    sy_model* mm = m;
    plan->ops.push_back([mm, c, x, y, res]() { return sy_conv_run(mm->ctx, c.id, x, y, res); });
    size_t s = conv_scratch_bytes(m->ctx->convs[c.id - 1].get(), x->n, x->h, x->w);
    if (s > plan->scratch) plan->scratch = s;
  }

  sy_tensor* conv_new(const Conv& c, sy_tensor* x) {
    int oh = 0, ow = 0;
    sy_conv_out_size(m->ctx, c.id, x->h, x->w, &oh, &ow);
    sy_tensor* y = alloc(x->n, c.oc, oh, ow);
    conv(c, x, y);
    return y;
  }

  // C2f (PtModel.cs:307) with chunk/concat as slices of one buffer and the
  // Bottleneck add (PtModel.cs:302-303) fused into the second conv.
  void c2f(const sy_model::C2f& f, sy_tensor* x, sy_tensor* out) {
    const int n = (int)f.m.size(), c = f.c;
    sy_tensor* buf = alloc(x->n, (2 + n) * c, x->h, x->w);
    conv(f.cv1, x, slice(buf, 0, 2 * c));
    for (int i = 0; i < n; ++i) {
      sy_tensor* prev = slice(buf, (1 + i) * c, c);
      sy_tensor* tmp = alloc(x->n, c, x->h, x->w);
      conv(f.m[i].first, prev, tmp);
      conv(f.m[i].second, tmp, slice(buf, (2 + i) * c, c), f.add ? prev : nullptr);
    }
    conv(f.cv2, buf, out);
  }

  // SPPF (PtModel.cs:310-311): cv1, three chained 5x5 pools, cv2 of the concat.
  void sppf(sy_tensor* x, sy_tensor* out) {
    const int c = m->s_cv1.oc;
    sy_tensor* buf = alloc(x->n, 4 * c, x->h, x->w);
    sy_tensor* s0 = slice(buf, 0, c);
    conv(m->s_cv1, x, s0);
    sy_tensor *s1 = slice(buf, c, c), *s2 = slice(buf, 2 * c, c), *s3 = slice(buf, 3 * c, c);
    sy_model* mm = m;
    plan->ops.push_back([mm, s0, s1, s2, s3]() { return sy_sppf_pool(mm->ctx, s0, s1, s2, s3); });
    conv(m->s_cv2, buf, out);
  }

  void upsample(sy_tensor* x, sy_tensor* out) {
    sy_model* mm = m;
    plan->ops.push_back([mm, x, out]() { return sy_resize_nearest(mm->ctx, x, out); });
  }

  void resolve(char* base) {
    for (auto& f : fixups) f.first->data = (float*)(base + f.second);
    for (auto& s : slices) {
      sy_tensor* t = std::get<0>(s);
      sy_tensor* parent = std::get<1>(s);
      t->data = parent->data + std::get<2>(s);
      t->ldc = parent->ldc;
    }
  }
};

int build_plan(sy_model* m, int B, int H, int W, Plan* plan) {
  SY_CHECK(B > 0 && H > 0 && W > 0 && H % 32 == 0 && W % 32 == 0, SY_EINVAL,
           "PT YOLO expects NCHW RGB with height/width multiples of 32 (got %dx%d)", H, W);
  plan->batch = B; plan->h = H; plan->w = W;
  Planner p{m, plan};
  const int nc = m->cfg.nc, reg = m->cfg.reg_max;
  const int h8 = H / 8, w8 = W / 8, h16 = H / 16, w16 = W / 16, h32 = H / 32, w32 = W / 32;
  const int anchors = h8 * w8 + h16 * w16 + h32 * w32;
  // Input and output live in the plan arena too.
  const size_t in_off = 0;
  p.used = (size_t)B * 3 * H * W * sizeof(float);
  p.used = (p.used + 255) & ~size_t(255);
  const size_t out_off = p.used;
  p.used += (size_t)B * (nc + 4) * anchors * sizeof(float);
  auto input = std::make_unique<sy_tensor>(sy_tensor{nullptr, B, 3, H, W, 3, SY_LAYOUT_NCHW});
  p.fixups.emplace_back(input.get(), in_off);
  sy_tensor* x = input.get();
  p.store.push_back(std::move(input));

  // Concat buffers first, so their inputs write in place.
  sy_tensor* cat11 = p.alloc(B, m->c1024 + m->c512, h16, w16);  // [up(L9), L6]
  sy_tensor* cat14 = p.alloc(B, m->c512 + m->c256, h8, w8);     // [up(L12), L4]
  sy_tensor* cat17 = p.alloc(B, m->c256 + m->c512, h16, w16);   // [L16, L12]
  sy_tensor* cat20 = p.alloc(B, m->c512 + m->c1024, h32, w32);  // [L19, L9]

  sy_tensor* t0 = p.conv_new(m->c0, x);
  sy_tensor* t1 = p.conv_new(m->c1, t0);
  sy_tensor* t2 = p.alloc(B, m->c128, t1->h, t1->w);
  p.c2f(m->f2, t1, t2);
  sy_tensor* t3 = p.conv_new(m->c3, t2);
  sy_tensor* l4 = p.slice(cat14, m->c512, m->c256);
  p.c2f(m->f4, t3, l4);
  sy_tensor* t5 = p.conv_new(m->c5, l4);
  sy_tensor* l6 = p.slice(cat11, m->c1024, m->c512);
  p.c2f(m->f6, t5, l6);
  sy_tensor* t7 = p.conv_new(m->c7, l6);
  sy_tensor* t8 = p.alloc(B, m->c1024, h32, w32);
  p.c2f(m->f8, t7, t8);
  sy_tensor* l9 = p.slice(cat20, m->c512, m->c1024);
  p.sppf(t8, l9);
  p.upsample(l9, p.slice(cat11, 0, m->c1024));
  sy_tensor* l12 = p.slice(cat17, m->c256, m->c512);
  p.c2f(m->f12, cat11, l12);
  p.upsample(l12, p.slice(cat14, 0, m->c512));
  sy_tensor* l15 = p.alloc(B, m->c256, h8, w8);
  p.c2f(m->f15, cat14, l15);
  p.conv(m->c16, l15, p.slice(cat17, 0, m->c256));
  sy_tensor* l18 = p.alloc(B, m->c512, h16, w16);
  p.c2f(m->f18, cat17, l18);
  p.conv(m->c19, l18, p.slice(cat20, 0, m->c512));
  sy_tensor* l21 = p.alloc(B, m->c1024, h32, w32);
  p.c2f(m->f21, cat20, l21);

  // Detect (PtModel.cs:444-504): per level box/class chains into one raw
  // head buffer [4*reg_max | nc], then one joined decode.
  sy_tensor* feats[3] = {l15, l18, l21};
  auto levels = std::make_shared<std::vector<sy_tensor*>>();
  for (int i = 0; i < 3; ++i) {
    sy_tensor* f = feats[i];
    const int c2 = m->box_ch, c3 = m->cls_ch;
    sy_tensor* a = p.alloc(B, c2 + c3, f->h, f->w);
    p.conv(m->head0[i], f, a);
    sy_tensor* b = p.alloc(B, c2 + c3, f->h, f->w);
    p.conv(m->box1[i], p.slice(a, 0, c2), p.slice(b, 0, c2));
    p.conv(m->cls1[i], p.slice(a, c2, c3), p.slice(b, c2, c3));
    sy_tensor* r = p.alloc(B, 4 * reg + nc, f->h, f->w);
    p.conv(m->box2[i], p.slice(b, 0, c2), p.slice(r, 0, 4 * reg));
    p.conv(m->cls2[i], p.slice(b, c2, c3), p.slice(r, 4 * reg, nc));
    levels->push_back(r);
  }
  {
    sy_model* mm = m;
    Plan* pl = plan;
    const int total = anchors;
    plan->ops.push_back([mm, pl, levels, total, nc, reg]() {
      sy_tensor lv[3] = {*(*levels)[0], *(*levels)[1], *(*levels)[2]};
      const float strides[3] = {8.f, 16.f, 32.f};
      return sy_detect_decode(mm->ctx, lv, strides, 3, reg, nc, 0, pl->output, total);
    });
  }

  // Allocate the arena and resolve every view.
  plan->bytes = p.used;
  SY_HIP(hipMalloc((void**)&plan->arena, plan->bytes));
  p.resolve(plan->arena);
  plan->input = (float*)(plan->arena + in_off);
  plan->output = (float*)(plan->arena + out_off);
  // Keep the views alive for the lifetime of the ops.
  auto keep = std::make_shared<std::vector<std::unique_ptr<sy_tensor>>>(std::move(p.store));
  plan->ops.push_back([keep]() { return SY_OK; });
  SY_TRY(ensure_scratch(m->ctx, plan->scratch));
  return SY_OK;
}

int get_plan(sy_model* m, int B, int H, int W, Plan** out) {
  auto key = std::make_tuple(B, H, W);
  auto it = m->plans.find(key);
  if (it == m->plans.end()) {
    auto plan = std::make_unique<Plan>();
    int rc = build_plan(m, B, H, W, plan.get());
    if (rc != SY_OK) {
      if (plan->arena) (void)hipFree(plan->arena);
      return rc;
    }
    it = m->plans.emplace(key, std::move(plan)).first;
  }
  *out = it->second.get();
  return SY_OK;
}

int run_ops(sy_model* m, Plan* plan) {
  for (auto& op : plan->ops) SY_TRY(op());
  (void)m;
  return SY_OK;
}

int run_plan(sy_model* m, Plan* plan) {
  sy_ctx* ctx = m->ctx;
  if (!m->use_graph || ctx->profiling) return run_ops(m, plan);
  if (!plan->graph) {
    // Capture on first use; ops must not allocate (scratch was reserved).
    SY_TRY(sy_graph_begin(ctx));
    int rc = run_ops(m, plan);
    uint64_t g = 0;
    int rc2 = sy_graph_end(ctx, &g);
    SY_TRY(rc);
    SY_TRY(rc2);
    plan->graph = g;
  }
  return sy_graph_launch(ctx, plan->graph);
}

}  // namespace

extern "C" {

int sy_model_layout(const sy_model_config* cfg, int32_t* out, int max_entries, int* count) {
  SY_TRY(validate_cfg(cfg));
  SY_CHECK(count, SY_EINVAL, "null count");
  ParamWalk pw;
  pw.layout = out;
  pw.max_entries = out ? max_entries : 0;
  V8Weights w;
  read_yolov8(pw, *cfg, w);
  *count = pw.count;
  return SY_OK;
}

int sy_model_create(sy_ctx* ctx, const sy_model_config* cfg, const float* params, size_t n_params, sy_model** out) {
  SY_CHECK(ctx && params && out, SY_EINVAL, "null argument");
  SY_TRY(validate_cfg(cfg));
  *out = nullptr;
  ParamWalk pw;
  pw.params = params;
  pw.n_params = n_params;
  V8Weights w;
  read_yolov8(pw, *cfg, w);
  SY_CHECK(!pw.overrun && pw.pos == n_params, SY_EINVAL, "parameter blob holds %zu floats, the model needs %zu",
           n_params, pw.pos);
  auto m = std::make_unique<sy_model>();
  m->ctx = ctx;
  m->cfg = *cfg;
  m->c64 = scale_ch(*cfg, 64); m->c128 = scale_ch(*cfg, 128); m->c256 = scale_ch(*cfg, 256);
  m->c512 = scale_ch(*cfg, 512); m->c1024 = scale_ch(*cfg, 1024);
  SY_TRY(make_conv(m.get(), w.c0, &m->c0));
  SY_TRY(make_conv(m.get(), w.c1, &m->c1));
  SY_TRY(make_conv(m.get(), w.c3, &m->c3));
  SY_TRY(make_conv(m.get(), w.c5, &m->c5));
  SY_TRY(make_conv(m.get(), w.c7, &m->c7));
  SY_TRY(make_conv(m.get(), w.c16, &m->c16));
  SY_TRY(make_conv(m.get(), w.c19, &m->c19));
  SY_TRY(make_conv(m.get(), w.s_cv1, &m->s_cv1));
  SY_TRY(make_conv(m.get(), w.s_cv2, &m->s_cv2));
  SY_TRY(make_c2f(m.get(), w.f2, &m->f2));
  SY_TRY(make_c2f(m.get(), w.f4, &m->f4));
  SY_TRY(make_c2f(m.get(), w.f6, &m->f6));
  SY_TRY(make_c2f(m.get(), w.f8, &m->f8));
  SY_TRY(make_c2f(m.get(), w.f12, &m->f12));
  SY_TRY(make_c2f(m.get(), w.f15, &m->f15));
  SY_TRY(make_c2f(m.get(), w.f18, &m->f18));
  SY_TRY(make_c2f(m.get(), w.f21, &m->f21));
  m->box_ch = w.box_ch;
  m->cls_ch = w.cls_ch;
  for (int i = 0; i < 3; ++i) {
    m->ch[i] = w.ch[i];
    // cv2[i][0] and cv3[i][0] read the same input: one conv, oc = c2 + c3.
    ConvW fused = w.box[i][0];
    fused.oc = w.box_ch + w.cls_ch;
    fused.w.insert(fused.w.end(), w.cls[i][0].w.begin(), w.cls[i][0].w.end());
    fused.b.insert(fused.b.end(), w.cls[i][0].b.begin(), w.cls[i][0].b.end());
    SY_TRY(make_conv(m.get(), fused, &m->head0[i]));
    SY_TRY(make_conv(m.get(), w.box[i][1], &m->box1[i]));
    SY_TRY(make_conv(m.get(), w.cls[i][1], &m->cls1[i]));
    SY_TRY(make_conv(m.get(), w.box[i][2], &m->box2[i]));
    SY_TRY(make_conv(m.get(), w.cls[i][2], &m->cls2[i]));
  }
  *out = m.release();
  return SY_OK;
}

void sy_model_destroy(sy_model* model) { delete model; }

int sy_model_output_shape(sy_model* m, int batch, int h, int w, int* channels, int* anchors) {
  SY_CHECK(m && channels && anchors, SY_EINVAL, "null argument");
  SY_CHECK(batch > 0 && h > 0 && w > 0 && h % 32 == 0 && w % 32 == 0, SY_EINVAL, "invalid input shape");
  *channels = m->cfg.nc + 4;
  *anchors = (h / 8) * (w / 8) + (h / 16) * (w / 16) + (h / 32) * (w / 32);
  return SY_OK;
}

int sy_model_buffers(sy_model* m, int batch, int h, int w, float** input, float** output) {
  SY_CHECK(m, SY_EINVAL, "null model");
  Plan* plan = nullptr;
  SY_TRY(get_plan(m, batch, h, w, &plan));
  if (input) *input = plan->input;
  if (output) *output = plan->output;
  return SY_OK;
}

int sy_model_run(sy_model* m, int batch, int h, int w) {
  SY_CHECK(m, SY_EINVAL, "null model");
  Plan* plan = nullptr;
  SY_TRY(get_plan(m, batch, h, w, &plan));
  return run_plan(m, plan);
}

int sy_model_predict_raw(sy_model* m, const float* input, int batch, int h, int w, float* out) {
  SY_CHECK(m && input && out, SY_EINVAL, "null argument");
  Plan* plan = nullptr;
  SY_TRY(get_plan(m, batch, h, w, &plan));
  sy_ctx* ctx = m->ctx;
  SY_HIP(hipMemcpyAsync(plan->input, input, (size_t)batch * 3 * h * w * sizeof(float), hipMemcpyHostToDevice,
                        ctx->stream));
  SY_TRY(run_plan(m, plan));
  int ch = 0, an = 0;
  SY_TRY(sy_model_output_shape(m, batch, h, w, &ch, &an));
  SY_HIP(hipMemcpyAsync(out, plan->output, (size_t)batch * ch * an * sizeof(float), hipMemcpyDeviceToHost,
                        ctx->stream));
  SY_HIP(hipStreamSynchronize(ctx->stream));
  return prof_collect(ctx);
}

int sy_model_set_graph(sy_model* m, int use_graph) {
  SY_CHECK(m, SY_EINVAL, "null model");
  m->use_graph = use_graph != 0;
  return SY_OK;
}

int sy_model_memory(sy_model* m, size_t* weight_bytes, size_t* arena_bytes) {
  SY_CHECK(m, SY_EINVAL, "null model");
  if (weight_bytes) *weight_bytes = m->weight_bytes;
  if (arena_bytes) {
    size_t s = 0;
    for (auto& kv : m->plans) s += kv.second->bytes;
    *arena_bytes = s + m->ctx->scratch_size;
  }
  return SY_OK;
}

}  // extern "C"
