// C++ host mirror of the reference's model interpreter (PtModel,
// src/SimdYolo/PtModel.cs) for the YOLOv8, YOLO11 and YOLO26 families
// (detect and segment):
//   * parameter walk in state_dict order + BN fold at load (PtModel.cs:84-145);
//   * a layer program with routing indices, as PtModel.Run walks it
//     (PtModel.cs:184-220), built from the ultralytics yolov8.yaml /
//     yolo11.yaml / yolo26.yaml topologies;
//   * module semantics of PtModel.Forward (PtModel.cs:267-359): Conv, C2f /
//     C3k2 (Bottleneck, C3k or Bottleneck + PSABlock inner blocks), SPPF
//     (with its pool count and shortcut), C2PSA / PSABlock / Attention,
//     Upsample, Concat; Detect (PtModel.cs:444-504) incl. the end-to-end
//     one2one head and its two-stage top-k with the mask coefficients as
//     extras (PtModel.cs:506-570); Segment / Segment26 with Proto / Proto26.
// Planned for MI355X:
//   * every activation is an NHWC view; each Concat buffer is allocated first
//     and its inputs' producers write straight into their channel slices;
//     C2f's chunk/concat are slices of one buffer, so no copies remain;
//   * residual adds (Bottleneck, PSABlock, Attention + pe) are fused into the
//     producing conv's epilogue;
//   * YOLOv8's first box and class convs share the level input and run as one
//     conv with concatenated output channels;
//   * a shape's op list is captured once into a hipGraph and replayed.
#include <algorithm>
#include <atomic>
#include <climits>
#include <cmath>
#include <condition_variable>
#include <cstring>
#include <functional>
#include <map>
#include <mutex>
#include <thread>
#include <tuple>

#include "host_copy.h"
#include "sy_internal.h"

using namespace sy;

namespace {

// ---------------------------------------------------------------- weights

struct ParamWalk {
  int32_t* layout = nullptr;
  int max_entries = 0;
  int count = 0;
  const float* params = nullptr;
  size_t n_params = 0, pos = 0;
  bool overrun = false;
  float eps = 1e-3f;

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

// Folded weights of one Conv (conv + BN [+ SiLU]) or Conv2d (+ bias).
struct ConvW {
  int ic = 0, oc = 0, k = 1, s = 1, g = 1;
  bool silu = true;
  std::vector<float> w, b;
};

// Conv(c1, c2, k, s, g, act): the BN fold of PtModel.Prepare.
ConvW read_conv(ParamWalk& pw, int ic, int oc, int k, int s, int g = 1, bool act = true) {
  ConvW c;
  c.ic = ic; c.oc = oc; c.k = k; c.s = s; c.g = g; c.silu = act;
  const int icg = ic / g;
  const float* w = pw.take(SY_P_CONV_WEIGHT, oc, icg, k, k, icg * k * k);
  const float* ga = pw.take(SY_P_BN_GAMMA, oc, 1, 1, 1, 0);
  const float* be = pw.take(SY_P_BN_BETA, oc, 1, 1, 1, 0);
  const float* mu = pw.take(SY_P_BN_MEAN, oc, 1, 1, 1, 0);
  const float* va = pw.take(SY_P_BN_VAR, oc, 1, 1, 1, 0);
  if (w && ga && be && mu && va) {
    c.w.resize((size_t)oc * icg * k * k);
    c.b.resize(oc);
    sy_fold_bn(w, oc, icg * k * k, nullptr, ga, be, mu, va, pw.eps, c.w.data(), c.b.data());
  }
  return c;
}

ConvW read_conv2d(ParamWalk& pw, int ic, int oc, int bias_kind) {
  ConvW c;
  c.ic = ic; c.oc = oc; c.silu = false;
  const float* w = pw.take(SY_P_CONV_WEIGHT, oc, ic, 1, 1, ic);
  const float* b = pw.take(bias_kind, oc, 1, 1, 1, 0);
  if (w && b) {
    c.w.assign(w, w + (size_t)oc * ic);
    c.b.assign(b, b + oc);
  }
  return c;
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

// ---------------------------------------------------------------- modules

struct Conv {
  uint64_t id = 0;
  int oc = 0;
};

struct Bottleneck {  // cv2(cv1(x)) [+ x]
  Conv cv1, cv2;
  bool add = false;
};

struct C3kM {  // cv3(cat(m(cv1(x)), cv2(x)))
  Conv cv1, cv2, cv3;
  std::vector<Bottleneck> m;
};

struct PsaM {
  Conv qkv, proj, pe, f0, f1;
  int heads = 0, kd = 0, hd = 0;
  float scale = 1.f;
};

struct C2fM {  // C2f / C3k2
  Conv cv1, cv2;
  int c = 0;
  std::vector<Bottleneck> b;
  std::vector<C3kM> k;
  std::vector<PsaM> a;  // with b: Sequential(Bottleneck, PSABlock) blocks
};

struct C2psaM {
  Conv cv1, cv2;
  int c = 0;
  std::vector<PsaM> m;
};

struct SppfM {
  Conv cv1, cv2;
  bool add = false;  // y + x (yolo26.yaml's SPPF shortcut)
};

struct DetectM {
  bool fused_first = false;          // YOLOv8: box[0] and cls[0] as one conv
  Conv first;                        // fused first conv (oc = box_ch + cls_ch)
  std::vector<Conv> box, cls;        // remaining convs of each branch
  int box_ch = 0, cls_ch = 0;
};

// Segment (PtModel.cs:353-360): Proto on the P3 feature (cv1 3x3, a 2x2
// stride-2 ConvTranspose2d, cv2 3x3, cv3 1x1 to nm) and per level the
// mask-coefficient branch cv4 (3x3, 3x3, Conv2d to nm).  Segment26 with
// Proto26 (PtModel.cs:345-352) first refines the P3 feature with the coarser
// levels, r = f0 + up2(refine0(f1)) + up4(refine1(f2)), and fuses it (3x3)
// before Proto's cv1.
struct SegM {
  Conv p_cv1, p_up, p_cv2, p_cv3;
  Conv cv4[3][3];
  bool proto26 = false;
  Conv refine[2], fuse;
  int nm = 0, npr = 0;
};

enum LayerType { L_CONV, L_C2F, L_SPPF, L_C2PSA, L_UP, L_CAT, L_DETECT };

struct Layer {
  LayerType type;
  std::vector<int> from;  // -1 = network input
  int c = 0;              // output channels
  Conv conv;
  C2fM c2f;
  SppfM sppf;
  C2psaM psa;
  DetectM det[3];
  SegM seg;  // nm > 0: Segment head
};

struct Builder {
  sy_model* m;
  ParamWalk pw;
  bool make;  // create device convs (false: layout enumeration only)
  int rc = SY_OK;
  size_t weight_bytes = 0;
  sy_ctx* ctx = nullptr;

  Conv mk(const ConvW& c) {
    Conv out;
    out.oc = c.oc;
    if (!make || rc != SY_OK) return out;
    const int p = c.k / 2;
    rc = sy_conv_create(ctx, c.w.data(), c.b.data(), c.oc, c.ic, c.k, c.k, c.s, c.s, p, p, p, p, 1, 1, c.g,
                        c.silu ? 1 : 0, &out.id);
    weight_bytes += (c.w.size() + c.b.size()) * sizeof(float);
    return out;
  }
  Conv conv(int ic, int oc, int k, int s, int g = 1, bool act = true) { return mk(read_conv(pw, ic, oc, k, s, g, act)); }
  Conv conv2d(int ic, int oc, int kind) { return mk(read_conv2d(pw, ic, oc, kind)); }
  // nn.ConvTranspose2d(ic, oc, 2, 2) with bias: weight [ic][oc][2][2].
  Conv up2(int ic, int oc) {
    const float* w = pw.take(SY_P_CONV_WEIGHT, ic, oc, 2, 2, oc * 4);
    const float* bias = pw.take(SY_P_BIAS, oc, 1, 1, 1, oc * 4);
    Conv out;
    out.oc = oc;
    if (!make || rc != SY_OK) return out;
    if (!w || !bias) {
      rc = SY_EINVAL;
      return out;
    }
    rc = sy_conv_transpose2x2_create(ctx, w, bias, ic, oc, &out.id);
    weight_bytes += ((size_t)ic * oc * 4 + oc) * sizeof(float);
    return out;
  }
  // Segment: Proto(ch0, npr, nm) then cv4 per level; c4 = max(ch0 / 4, nm).
  void segment(const sy_model_config& cfg, const int ch[3], SegM& sg) {
    sg.nm = cfg.nm;
    sg.npr = scale_ch(cfg, cfg.npr);
    sg.p_cv1 = conv(ch[0], sg.npr, 3, 1);
    sg.p_up = up2(sg.npr, sg.npr);
    sg.p_cv2 = conv(sg.npr, sg.npr, 3, 1);
    sg.p_cv3 = conv(sg.npr, cfg.nm, 1, 1);
    const int c4 = ch[0] / 4 > cfg.nm ? ch[0] / 4 : cfg.nm;
    for (int i = 0; i < 3; ++i) {
      sg.cv4[i][0] = conv(ch[i], c4, 3, 1);
      sg.cv4[i][1] = conv(c4, c4, 3, 1);
      sg.cv4[i][2] = conv2d(c4, cfg.nm, SY_P_BIAS);
    }
  }

  // Segment26: Proto(c_, c_, nm) then feat_refine / feat_fuse (Proto26's
  // registration order), then one2one_cv4 per level.
  void segment26(const sy_model_config& cfg, const int ch[3], SegM& sg) {
    sg.nm = cfg.nm;
    sg.npr = scale_ch(cfg, cfg.npr);
    sg.proto26 = true;
    sg.p_cv1 = conv(sg.npr, sg.npr, 3, 1);
    sg.p_up = up2(sg.npr, sg.npr);
    sg.p_cv2 = conv(sg.npr, sg.npr, 3, 1);
    sg.p_cv3 = conv(sg.npr, cfg.nm, 1, 1);
    sg.refine[0] = conv(ch[1], ch[0], 1, 1);
    sg.refine[1] = conv(ch[2], ch[0], 1, 1);
    sg.fuse = conv(ch[0], sg.npr, 3, 1);
    const int c4 = ch[0] / 4 > cfg.nm ? ch[0] / 4 : cfg.nm;
    for (int i = 0; i < 3; ++i) {
      sg.cv4[i][0] = conv(ch[i], c4, 3, 1);
      sg.cv4[i][1] = conv(c4, c4, 3, 1);
      sg.cv4[i][2] = conv2d(c4, cfg.nm, SY_P_BIAS);
    }
  }

  Bottleneck bottleneck(int c1, int c2, bool shortcut, double e) {
    Bottleneck b;
    const int c_ = (int)(c2 * e);
    b.cv1 = conv(c1, c_, 3, 1);
    b.cv2 = conv(c_, c2, 3, 1);
    b.add = shortcut && c1 == c2;
    return b;
  }
  C3kM c3k(int c1, int c2, int n, bool shortcut) {
    C3kM m3;
    const int c_ = (int)(c2 * 0.5);
    m3.cv1 = conv(c1, c_, 1, 1);
    m3.cv2 = conv(c1, c_, 1, 1);
    m3.cv3 = conv(2 * c_, c2, 1, 1);
    for (int i = 0; i < n; ++i) m3.m.push_back(bottleneck(c_, c_, shortcut, 1.0));
    return m3;
  }
  // C2f(c1, c2, n, shortcut): Bottleneck(c, c, e=1.0).  C3k2(c1, c2, n, c3k, e):
  // C3k(c, c, 2) or Bottleneck(c, c, e=0.5), shortcut on.  state_dict order:
  // cv1, cv2, m.*.
  C2fM c2f(int c1, int c2, int n, bool shortcut, double e, bool c3k2, bool use_c3k) {
    C2fM f;
    f.c = (int)(c2 * e);
    f.cv1 = conv(c1, 2 * f.c, 1, 1);
    f.cv2 = conv((2 + n) * f.c, c2, 1, 1);
    for (int i = 0; i < n; ++i) {
      if (c3k2 && use_c3k) f.k.push_back(c3k(f.c, f.c, 2, true));
      else f.b.push_back(bottleneck(f.c, f.c, c3k2 ? true : shortcut, c3k2 ? 0.5 : 1.0));
    }
    return f;
  }
  // SPPF(c1, c2, k=5, n=3, shortcut): yolo26.yaml's cv1 has no activation
  // and the output adds the input when c1 == c2.
  SppfM sppf(int c1, int c2, bool cv1_act = true, bool shortcut = false) {
    SppfM s;
    s.cv1 = conv(c1, c1 / 2, 1, 1, 1, cv1_act);
    s.cv2 = conv(c1 / 2 * 4, c2, 1, 1);
    s.add = shortcut && c1 == c2;
    return s;
  }
  // PSABlock(c, attn_ratio 0.5, heads): Attention (qkv, proj, pe), then the
  // ffn Conv(c, 2c, 1), Conv(2c, c, 1, act=False).
  PsaM psa(int c, int heads) {
    PsaM b;
    b.heads = heads;
    b.hd = c / b.heads;
    b.kd = (int)(b.hd * 0.5);
    b.scale = 1.0f / std::sqrt((float)b.kd);
    const int h = c + 2 * b.kd * b.heads;
    b.qkv = conv(c, h, 1, 1, 1, false);
    b.proj = conv(c, c, 1, 1, 1, false);
    b.pe = conv(c, c, 3, 1, c, false);
    b.f0 = conv(c, 2 * c, 1, 1);
    b.f1 = conv(2 * c, c, 1, 1, 1, false);
    return b;
  }
  // C3k2(c1, c2, n, e, attn=True): inner blocks Sequential(Bottleneck(c, c,
  // e=0.5), PSABlock(c, 0.5, max(c / 64, 1))).
  C2fM c2f_attn(int c1, int c2, int n, double e) {
    C2fM f;
    f.c = (int)(c2 * e);
    f.cv1 = conv(c1, 2 * f.c, 1, 1);
    f.cv2 = conv((2 + n) * f.c, c2, 1, 1);
    for (int i = 0; i < n; ++i) {
      f.b.push_back(bottleneck(f.c, f.c, true, 0.5));
      f.a.push_back(psa(f.c, f.c / 64 > 1 ? f.c / 64 : 1));
    }
    return f;
  }
  C2psaM c2psa(int c1, int n) {
    C2psaM p;
    p.c = (int)(c1 * 0.5);
    p.cv1 = conv(c1, 2 * p.c, 1, 1);
    p.cv2 = conv(2 * p.c, c1, 1, 1);
    for (int i = 0; i < n; ++i) p.m.push_back(psa(p.c, p.c / 64));
    return p;
  }
  // Detect: cv2 (box) for every level, then cv3 (class) for every level.
  void detect(const sy_model_config& cfg, const int ch[3], bool dw_cls, DetectM det[3]) {
    int c2 = 16;
    if (ch[0] / 4 > c2) c2 = ch[0] / 4;
    if (4 * cfg.reg_max > c2) c2 = 4 * cfg.reg_max;
    int c3 = cfg.nc < 100 ? cfg.nc : 100;
    if (ch[0] > c3) c3 = ch[0];
    ConvW first_box[3];
    for (int i = 0; i < 3; ++i) {
      det[i].box_ch = c2;
      det[i].cls_ch = c3;
      if (!dw_cls) {
        first_box[i] = read_conv(pw, ch[i], c2, 3, 1);
      } else {
        det[i].box.push_back(conv(ch[i], c2, 3, 1));
      }
      det[i].box.push_back(conv(c2, c2, 3, 1));
      det[i].box.push_back(conv2d(c2, 4 * cfg.reg_max, SY_P_BIAS_BOX));
    }
    for (int i = 0; i < 3; ++i) {
      if (!dw_cls) {
        ConvW cls0 = read_conv(pw, ch[i], c3, 3, 1);
        ConvW fused = first_box[i];
        fused.oc = c2 + c3;
        fused.w.insert(fused.w.end(), cls0.w.begin(), cls0.w.end());
        fused.b.insert(fused.b.end(), cls0.b.begin(), cls0.b.end());
        det[i].fused_first = true;
        det[i].first = mk(fused);
        det[i].cls.push_back(conv(c3, c3, 3, 1));
      } else {
        det[i].cls.push_back(conv(ch[i], ch[i], 3, 1, ch[i]));  // DWConv(x, x, 3)
        det[i].cls.push_back(conv(ch[i], c3, 1, 1));
        det[i].cls.push_back(conv(c3, c3, 3, 1, c3));  // DWConv(c3, c3, 3)
        det[i].cls.push_back(conv(c3, c3, 1, 1));
      }
      det[i].cls.push_back(conv2d(c3, cfg.nc, SY_P_BIAS_CLS));
    }
  }
};

Layer L(LayerType t, std::vector<int> from, int c) {
  Layer l;
  l.type = t;
  l.from = std::move(from);
  l.c = c;
  return l;
}

// ultralytics yolov8.yaml.
void build_yolov8(Builder& b, const sy_model_config& cfg, std::vector<Layer>& ls) {
  const int c64 = scale_ch(cfg, 64), c128 = scale_ch(cfg, 128), c256 = scale_ch(cfg, 256), c512 = scale_ch(cfg, 512),
            c1024 = scale_ch(cfg, 1024);
  const int n3 = scale_n(cfg, 3), n6 = scale_n(cfg, 6);
  auto conv = [&](int from, int c1, int c2, int s) {
    Layer l = L(L_CONV, {from}, c2);
    l.conv = b.conv(c1, c2, 3, s);
    ls.push_back(l);
  };
  auto c2f = [&](int from, int c1, int c2, int n, bool sc) {
    Layer l = L(L_C2F, {from}, c2);
    l.c2f = b.c2f(c1, c2, n, sc, 0.5, false, false);
    ls.push_back(l);
  };
  conv(-1, 3, c64, 2);                 // 0
  conv(0, c64, c128, 2);               // 1
  c2f(1, c128, c128, n3, true);        // 2
  conv(2, c128, c256, 2);              // 3
  c2f(3, c256, c256, n6, true);        // 4
  conv(4, c256, c512, 2);              // 5
  c2f(5, c512, c512, n6, true);        // 6
  conv(6, c512, c1024, 2);             // 7
  c2f(7, c1024, c1024, n3, true);      // 8
  {
    Layer l = L(L_SPPF, {8}, c1024);   // 9
    l.sppf = b.sppf(c1024, c1024);
    ls.push_back(l);
  }
  ls.push_back(L(L_UP, {9}, c1024));                   // 10
  ls.push_back(L(L_CAT, {10, 6}, c1024 + c512));       // 11
  c2f(11, c1024 + c512, c512, n3, false);              // 12
  ls.push_back(L(L_UP, {12}, c512));                   // 13
  ls.push_back(L(L_CAT, {13, 4}, c512 + c256));        // 14
  c2f(14, c512 + c256, c256, n3, false);               // 15
  conv(15, c256, c256, 2);                             // 16
  ls.push_back(L(L_CAT, {16, 12}, c256 + c512));       // 17
  c2f(17, c256 + c512, c512, n3, false);               // 18
  conv(18, c512, c512, 2);                             // 19
  ls.push_back(L(L_CAT, {19, 9}, c512 + c1024));       // 20
  c2f(20, c512 + c1024, c1024, n3, false);             // 21
  Layer d = L(L_DETECT, {15, 18, 21}, cfg.nc + 4);     // 22
  const int ch[3] = {c256, c512, c1024};
  b.detect(cfg, ch, false, d.det);
  if (cfg.nm > 0) b.segment(cfg, ch, d.seg);
  ls.push_back(d);
}

// ultralytics yolo11.yaml.
void build_yolo11(Builder& b, const sy_model_config& cfg, std::vector<Layer>& ls) {
  const int c64 = scale_ch(cfg, 64), c128 = scale_ch(cfg, 128), c256 = scale_ch(cfg, 256), c512 = scale_ch(cfg, 512),
            c1024 = scale_ch(cfg, 1024);
  const int n2 = scale_n(cfg, 2);
  // The m/l/x scales (width >= 1) build every C3k2 with C3k blocks.
  const bool all_c3k = cfg.width >= 1.0;
  auto conv = [&](int from, int c1, int c2, int s) {
    Layer l = L(L_CONV, {from}, c2);
    l.conv = b.conv(c1, c2, 3, s);
    ls.push_back(l);
  };
  auto c3k2 = [&](int from, int c1, int c2, bool c3k, double e) {
    Layer l = L(L_C2F, {from}, c2);
    l.c2f = b.c2f(c1, c2, n2, true, e, true, c3k || all_c3k);
    ls.push_back(l);
  };
  conv(-1, 3, c64, 2);                       // 0
  conv(0, c64, c128, 2);                     // 1
  c3k2(1, c128, c256, false, 0.25);          // 2
  conv(2, c256, c256, 2);                    // 3
  c3k2(3, c256, c512, false, 0.25);          // 4
  conv(4, c512, c512, 2);                    // 5
  c3k2(5, c512, c512, true, 0.5);            // 6
  conv(6, c512, c1024, 2);                   // 7
  c3k2(7, c1024, c1024, true, 0.5);          // 8
  {
    Layer l = L(L_SPPF, {8}, c1024);         // 9
    l.sppf = b.sppf(c1024, c1024);
    ls.push_back(l);
  }
  {
    Layer l = L(L_C2PSA, {9}, c1024);        // 10
    l.psa = b.c2psa(c1024, n2);
    ls.push_back(l);
  }
  ls.push_back(L(L_UP, {10}, c1024));                  // 11
  ls.push_back(L(L_CAT, {11, 6}, c1024 + c512));       // 12
  c3k2(12, c1024 + c512, c512, false, 0.5);            // 13
  ls.push_back(L(L_UP, {13}, c512));                   // 14
  ls.push_back(L(L_CAT, {14, 4}, c512 + c512));        // 15
  c3k2(15, c512 + c512, c256, false, 0.5);             // 16
  conv(16, c256, c256, 2);                             // 17
  ls.push_back(L(L_CAT, {17, 13}, c256 + c512));       // 18
  c3k2(18, c256 + c512, c512, false, 0.5);             // 19
  conv(19, c512, c512, 2);                             // 20
  ls.push_back(L(L_CAT, {20, 10}, c512 + c1024));      // 21
  c3k2(21, c512 + c1024, c1024, true, 0.5);            // 22
  Layer d = L(L_DETECT, {16, 19, 22}, cfg.nc + 4);     // 23
  const int ch[3] = {c256, c512, c1024};
  b.detect(cfg, ch, true, d.det);
  if (cfg.nm > 0) b.segment(cfg, ch, d.seg);
  ls.push_back(d);
}

// ultralytics yolo26.yaml / yolo26-seg.yaml: the YOLO11 backbone with an
// SPPF whose cv1 has no activation, n = 3 pools and a shortcut; head C3k2
// blocks with C3k inner blocks, the last with attention blocks; the
// end-to-end Detect (one2one_cv2 / one2one_cv3, PtModel.cs:449-450; reg_max
// 1 in the published scales) and Segment26 (one2one_cv4, Proto26).
void build_yolo26(Builder& b, const sy_model_config& cfg, std::vector<Layer>& ls) {
  const int c64 = scale_ch(cfg, 64), c128 = scale_ch(cfg, 128), c256 = scale_ch(cfg, 256), c512 = scale_ch(cfg, 512),
            c1024 = scale_ch(cfg, 1024);
  const int n2 = scale_n(cfg, 2);
  const bool all_c3k = cfg.width >= 1.0;
  auto conv = [&](int from, int c1, int c2, int s) {
    Layer l = L(L_CONV, {from}, c2);
    l.conv = b.conv(c1, c2, 3, s);
    ls.push_back(l);
  };
  auto c3k2 = [&](int from, int c1, int c2, bool c3k, double e) {
    Layer l = L(L_C2F, {from}, c2);
    l.c2f = b.c2f(c1, c2, n2, true, e, true, c3k || all_c3k);
    ls.push_back(l);
  };
  conv(-1, 3, c64, 2);                       // 0
  conv(0, c64, c128, 2);                     // 1
  c3k2(1, c128, c256, false, 0.25);          // 2
  conv(2, c256, c256, 2);                    // 3
  c3k2(3, c256, c512, false, 0.25);          // 4
  conv(4, c512, c512, 2);                    // 5
  c3k2(5, c512, c512, true, 0.5);            // 6
  conv(6, c512, c1024, 2);                   // 7
  c3k2(7, c1024, c1024, true, 0.5);          // 8
  {
    Layer l = L(L_SPPF, {8}, c1024);         // 9
    l.sppf = b.sppf(c1024, c1024, false, true);
    ls.push_back(l);
  }
  {
    Layer l = L(L_C2PSA, {9}, c1024);        // 10
    l.psa = b.c2psa(c1024, n2);
    ls.push_back(l);
  }
  ls.push_back(L(L_UP, {10}, c1024));                  // 11
  ls.push_back(L(L_CAT, {11, 6}, c1024 + c512));       // 12
  c3k2(12, c1024 + c512, c512, true, 0.5);             // 13
  ls.push_back(L(L_UP, {13}, c512));                   // 14
  ls.push_back(L(L_CAT, {14, 4}, c512 + c512));        // 15
  c3k2(15, c512 + c512, c256, true, 0.5);              // 16
  conv(16, c256, c256, 2);                             // 17
  ls.push_back(L(L_CAT, {17, 13}, c256 + c512));       // 18
  c3k2(18, c256 + c512, c512, true, 0.5);              // 19
  conv(19, c512, c512, 2);                             // 20
  ls.push_back(L(L_CAT, {20, 10}, c512 + c1024));      // 21
  {
    Layer l = L(L_C2F, {21}, c1024);                   // 22
    l.c2f = b.c2f_attn(c512 + c1024, c1024, scale_n(cfg, 1), 0.5);
    ls.push_back(l);
  }
  Layer d = L(L_DETECT, {16, 19, 22}, cfg.nc + 4);     // 23
  const int ch[3] = {c256, c512, c1024};
  b.detect(cfg, ch, true, d.det);
  if (cfg.nm > 0) b.segment26(cfg, ch, d.seg);
  ls.push_back(d);
}

// Rows the end-to-end head keeps (Detect.max_det, read by PtModel.cs:506,
// 530 with default 300).
constexpr int kEndToEndMaxDet = 300;

bool end_to_end(const sy_model_config& cfg) { return cfg.arch == SY_ARCH_YOLO26; }

int validate_cfg(const sy_model_config* cfg) {
  SY_CHECK(cfg, SY_EINVAL, "null model config");
  SY_CHECK(cfg->arch == SY_ARCH_YOLOV8 || cfg->arch == SY_ARCH_YOLO11 || cfg->arch == SY_ARCH_YOLO26, SY_EUNSUPPORTED,
           "unsupported architecture %d", cfg->arch);
  SY_CHECK(cfg->depth > 0 && cfg->width > 0 && cfg->max_channels > 0 && cfg->nc > 0 && cfg->reg_max > 0 &&
               cfg->bn_eps > 0 && cfg->nm >= 0 && (cfg->nm == 0 || cfg->npr > 0),
           SY_EINVAL, "invalid model config");
  return SY_OK;
}

void build_layers(Builder& b, const sy_model_config& cfg, std::vector<Layer>& ls) {
  if (cfg.arch == SY_ARCH_YOLO26) build_yolo26(b, cfg, ls);
  else if (cfg.arch == SY_ARCH_YOLO11) build_yolo11(b, cfg, ls);
  else build_yolov8(b, cfg, ls);
}

// ---------------------------------------------------------------- planning

struct Plan {
  int batch = 0, h = 0, w = 0;
  char* arena = nullptr;
  size_t bytes = 0;           // the arena, with activation buffers shared by liveness
  size_t unshared_bytes = 0;  // what it would take with every buffer separate
  float* input = nullptr;   // [B,3,H,W] NCHW
  float* head = nullptr;    // [B,nc+4(+nm),A] joined, decoded head
  float* output = nullptr;  // the head, or for end-to-end models the selected rows [B,k,6(+nm)]
  float* proto = nullptr;   // Segment: [B,nm,H/4,W/4] NCHW
  // Enqueued in order.  An op of lane k >= 1 belongs to a branch that only
  // depends on the main chain up to the fork of level k.  A graph captured
  // with branch level L runs the ops of lanes 1..L on the context's side
  // stream (forked from and joined back to the main stream by events);
  // otherwise every op runs in order on the main stream.
  enum Kind { kOp, kFork, kJoin };
  struct Op {
    int kind = kOp, lane = 0;
    std::function<int()> f;
  };
  std::vector<Op> ops;
  static constexpr int kMaxLevel = 2;
  hipEvent_t fork_ev[kMaxLevel] = {nullptr, nullptr}, join_ev = nullptr;
  uint64_t graph = 0;
  int level = 0;  // branch level of the kept graph (chosen by timing)
  // A single-stream capture of the same ops, for callers that launch the
  // forward behind cross-stream waits (the host I/O pipeline): launching a
  // branched graph there blocks the host until the graph has nearly run,
  // which would serialise the copies with the forward.
  uint64_t graph0 = 0;
  size_t scratch = 0;
  bool warmed = false;  // an eager pass has run (and tuned the convolutions)
};

}  // namespace

namespace {

// Staging of sy_model_predict_raw / _seg: pinned host rings (the caller's
// buffers are pageable; DMA runs at full PCIe rate only from pinned memory),
// device buffers for two batch chunks in flight, a stream each way, events.
struct HostIO {
  static constexpr size_t kPiece = size_t(8) << 20;  // bytes per pinned slot
  static constexpr int kSlots = 3;                   // slots per direction
  hipStream_t up = nullptr, down = nullptr;
  char* pin_in[kSlots] = {};
  char* pin_out[kSlots] = {};
  hipEvent_t in_slot[kSlots] = {}, out_slot[kSlots] = {};
  bool in_slot_used[kSlots] = {};
  char* dev_in[2] = {};
  char* dev_out[2] = {};
  size_t dev_in_bytes = 0, dev_out_bytes = 0;
  hipEvent_t in_ready[2] = {}, in_free[2] = {}, out_ready[2] = {}, out_free[2] = {};
  bool in_free_rec[2] = {}, out_free_rec[2] = {};
  std::unique_ptr<CopyPool> pool, pool_down;  // host copies up / down (separate: both run at once)
  ~HostIO() {
    if (up) (void)hipStreamSynchronize(up);
    if (down) (void)hipStreamSynchronize(down);
    for (int i = 0; i < kSlots; ++i) {
      if (pin_in[i]) (void)hipHostFree(pin_in[i]);
      if (pin_out[i]) (void)hipHostFree(pin_out[i]);
      if (in_slot[i]) (void)hipEventDestroy(in_slot[i]);
      if (out_slot[i]) (void)hipEventDestroy(out_slot[i]);
    }
    for (int i = 0; i < 2; ++i) {
      if (dev_in[i]) (void)hipFree(dev_in[i]);
      if (dev_out[i]) (void)hipFree(dev_out[i]);
      for (hipEvent_t e : {in_ready[i], in_free[i], out_ready[i], out_free[i]})
        if (e) (void)hipEventDestroy(e);
    }
    if (up) (void)hipStreamDestroy(up);
    if (down) (void)hipStreamDestroy(down);
  }
};

}  // namespace

struct sy_model {
  sy_ctx* ctx = nullptr;
  std::unique_ptr<HostIO> io;
  sy_model_config cfg{};
  bool use_graph = true;
  int branch_level = -1;  // -1: chosen per plan by timing
  size_t weight_bytes = 0;
  std::vector<Layer> layers;
  std::map<std::tuple<int, int, int>, std::unique_ptr<Plan>> plans;
  ~sy_model() {
    if (!ctx) return;
    (void)hipStreamSynchronize(ctx->stream);
    io.reset();
    for (auto& kv : plans) {
      if (kv.second->graph) sy_graph_destroy(ctx, kv.second->graph);
      if (kv.second->graph0) sy_graph_destroy(ctx, kv.second->graph0);
      if (kv.second->arena) (void)hipFree(kv.second->arena);
      for (hipEvent_t e : kv.second->fork_ev)
        if (e) (void)hipEventDestroy(e);
      if (kv.second->join_ev) (void)hipEventDestroy(kv.second->join_ev);
    }
  }
};

namespace {

// Activation buffers of a plan share the arena by liveness: every op names
// the buffers it reads or writes, a buffer holds its data from its first to
// its last op, and buffers whose op intervals are disjoint may take the same
// bytes.  Ops run in list order on one stream, except the ops of a graph
// branch (lane k >= 1), which may run anywhere between the branch's fork and
// the join: a buffer a branch op touches is kept from that fork (or its
// first op, if earlier) to the join, so it never shares bytes with a buffer
// of the concurrently running main chain.  The input, head, output and
// prototype buffers sit below the shared region and are never reused.
struct Planner {
  sy_model* m;
  Plan* plan;
  size_t used = 0;  // fixed region (input, head, output, prototypes)
  struct Buf {
    size_t size = 0;
    int first = INT_MAX, last = -1;  // op indices
    unsigned lanes = 0;              // bit k: touched by an op of branch lane k
    size_t off = 0;
  };
  std::vector<Buf> bufs;
  std::map<const sy_tensor*, int> root;  // view -> the buffer it lies in
  std::vector<std::pair<sy_tensor*, size_t>> fixed;  // tensors at fixed arena offsets
  std::vector<std::pair<sy_tensor*, int>> fixups;    // tensors at the start of a shared buffer
  std::vector<std::tuple<sy_tensor*, sy_tensor*, int>> slices;
  std::vector<std::unique_ptr<sy_tensor>> store;

  sy_tensor* alloc(int n, int c, int h, int w) {
    auto t = std::make_unique<sy_tensor>(sy_tensor{nullptr, n, c, h, w, c, SY_LAYOUT_NHWC});
    const int id = (int)bufs.size();
    bufs.push_back(Buf{(size_t)n * c * h * w * sizeof(float)});
    fixups.emplace_back(t.get(), id);
    root[t.get()] = id;
    store.push_back(std::move(t));
    return store.back().get();
  }
  sy_tensor* slice(sy_tensor* parent, int c0, int cn) {
    auto t = std::make_unique<sy_tensor>(*parent);
    t->c = cn;
    slices.emplace_back(t.get(), parent, c0);
    auto r = root.find(parent);
    if (r != root.end()) root[t.get()] = r->second;
    store.push_back(std::move(t));
    return store.back().get();
  }
  int lane = 0;  // lane of the ops added now
  // An op and the views it reads or writes (views in the fixed region, or
  // null, are ignored).
  void op(std::function<int()> f, std::initializer_list<const sy_tensor*> uses) {
    const int k = (int)plan->ops.size();
    for (const sy_tensor* t : uses) {
      auto r = t ? root.find(t) : root.end();
      if (r == root.end()) continue;
      Buf& b = bufs[r->second];
      b.first = std::min(b.first, k);
      b.last = std::max(b.last, k);
      if (lane > 0) b.lanes |= 1u << lane;
    }
    plan->ops.push_back(Plan::Op{Plan::kOp, lane, std::move(f)});
  }
  // Offsets of the shared buffers above `base` (greedy, largest first: each
  // takes the lowest 256-byte-aligned gap among the buffers it overlaps in
  // time).  Returns the arena size.
  size_t pack(size_t base) {
    int fork_at[Plan::kMaxLevel + 1], join_at = (int)plan->ops.size();
    for (int& f : fork_at) f = -1;
    for (size_t k = 0; k < plan->ops.size(); ++k) {
      const Plan::Op& o = plan->ops[k];
      if (o.kind == Plan::kFork && o.lane >= 1 && o.lane <= Plan::kMaxLevel) fork_at[o.lane] = (int)k;
      if (o.kind == Plan::kJoin) join_at = (int)k;
    }
    for (Buf& b : bufs)
      for (int l = 1; l <= Plan::kMaxLevel; ++l)
        if (b.lanes & (1u << l)) {
          if (fork_at[l] >= 0) b.first = std::min(b.first, fork_at[l]);
          b.last = std::max(b.last, join_at);
        }
    std::vector<int> order(bufs.size());
    for (size_t i = 0; i < order.size(); ++i) order[i] = (int)i;
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return bufs[a].size > bufs[b].size; });
    auto align = [](size_t v) { return (v + 255) & ~size_t(255); };
    size_t end = base;
    std::vector<int> placed;
    for (int id : order) {
      Buf& b = bufs[id];
      if (b.last < 0) {  // no op touches it
        b.off = align(base);
        end = std::max(end, b.off + b.size);
        continue;
      }
      std::vector<int> live;
      for (int q : placed)
        if (bufs[q].first <= b.last && b.first <= bufs[q].last) live.push_back(q);
      std::sort(live.begin(), live.end(), [&](int a, int c) { return bufs[a].off < bufs[c].off; });
      size_t at = align(base);
      for (int q : live) {
        if (at + b.size <= bufs[q].off) break;
        at = std::max(at, align(bufs[q].off + bufs[q].size));
      }
      b.off = at;
      end = std::max(end, at + b.size);
      placed.push_back(id);
    }
    return end;
  }
  // Bytes the shared buffers would take without reuse.
  size_t unshared() const {
    size_t s = 0;
    for (const Buf& b : bufs) s += (b.size + 255) & ~size_t(255);
    return s;
  }
  void fork(int level) { plan->ops.push_back(Plan::Op{Plan::kFork, level, nullptr}); }
  void join() { plan->ops.push_back(Plan::Op{Plan::kJoin, 0, nullptr}); }
  void reserve(size_t s) {
    if (s > plan->scratch) plan->scratch = s;
  }

  void conv(const Conv& c, sy_tensor* x, sy_tensor* y, sy_tensor* res = nullptr) {
    sy_ctx* ctx = m->ctx;
    op([ctx, c, x, y, res]() { return sy_conv_run(ctx, c.id, x, y, res); }, {x, y, res});
    reserve(conv_scratch_bytes(ctx->convs[c.id - 1].get(), x->n, x->h, x->w));
  }
  void conv_upsampled(const Conv& c, sy_tensor* xu, sy_tensor* x, sy_tensor* y) {
    sy_ctx* ctx = m->ctx;
    ConvPlan* cp = ctx->convs[c.id - 1].get();
    op([ctx, cp, xu, x, y]() { return conv_run_upsampled(ctx, cp, xu, x, y, nullptr); }, {xu, x, y});
    reserve(conv_scratch_bytes(cp, x->n, x->h, x->w));
  }
  sy_tensor* conv_new(const Conv& c, sy_tensor* x) {
    int oh = 0, ow = 0;
    sy_conv_out_size(m->ctx, c.id, x->h, x->w, &oh, &ow);
    sy_tensor* y = alloc(x->n, c.oc, oh, ow);
    conv(c, x, y);
    return y;
  }
  // Bottleneck (PtModel.cs:302-303), add fused into cv2.
  void bottleneck(const Bottleneck& b, sy_tensor* x, sy_tensor* out) {
    sy_tensor* t = alloc(x->n, b.cv1.oc, x->h, x->w);
    conv(b.cv1, x, t);
    conv(b.cv2, t, out, b.add ? x : nullptr);
  }
  // C3k (PtModel.cs:312): cv3(cat(m(cv1(x)), cv2(x))), the concat in place.
  void c3k(const C3kM& k, sy_tensor* x, sy_tensor* out) {
    const int c_ = k.cv1.oc;
    sy_tensor* buf = alloc(x->n, 2 * c_, x->h, x->w);
    sy_tensor* a = slice(buf, 0, c_);
    if (k.m.empty()) {
      conv(k.cv1, x, a);
    } else {
      sy_tensor* cur = alloc(x->n, c_, x->h, x->w);
      conv(k.cv1, x, cur);
      for (size_t i = 0; i < k.m.size(); ++i) {
        sy_tensor* dst = i + 1 == k.m.size() ? a : alloc(x->n, c_, x->h, x->w);
        bottleneck(k.m[i], cur, dst);
        cur = dst;
      }
    }
    conv(k.cv2, x, slice(buf, c_, c_));
    conv(k.cv3, buf, out);
  }
  // C2f / C3k2 (PtModel.cs:307): chunk/concat as slices of one buffer.
  // xu: when set, x's leading xu->c channels are the 2x nearest upsample of
  // xu and were not written; cv1 reads them from xu.
  void c2f(const C2fM& f, sy_tensor* x, sy_tensor* out, sy_tensor* xu = nullptr) {
    const int n = (int)(f.b.size() + f.k.size()), c = f.c;
    sy_tensor* buf = alloc(x->n, (2 + n) * c, x->h, x->w);
    if (xu)
      conv_upsampled(f.cv1, xu, x, slice(buf, 0, 2 * c));
    else
      conv(f.cv1, x, slice(buf, 0, 2 * c));
    for (int i = 0; i < n; ++i) {
      sy_tensor* prev = slice(buf, (1 + i) * c, c);
      sy_tensor* dst = slice(buf, (2 + i) * c, c);
      if (!f.k.empty()) {
        c3k(f.k[i], prev, dst);
      } else if (!f.a.empty()) {
        sy_tensor* t = alloc(x->n, c, x->h, x->w);
        bottleneck(f.b[i], prev, t);
        psa_block(f.a[i], t, dst);
      } else {
        bottleneck(f.b[i], prev, dst);
      }
    }
    conv(f.cv2, buf, out);
  }
  // SPPF (PtModel.cs:310-311): cv1, three chained 5x5 pools, cv2 of the concat.
  void sppf(const SppfM& s, sy_tensor* x, sy_tensor* out) {
    const int c = s.cv1.oc;
    sy_tensor* buf = alloc(x->n, 4 * c, x->h, x->w);
    sy_tensor* s0 = slice(buf, 0, c);
    conv(s.cv1, x, s0);
    sy_tensor *s1 = slice(buf, c, c), *s2 = slice(buf, 2 * c, c), *s3 = slice(buf, 3 * c, c);
    sy_ctx* ctx = m->ctx;
    op([ctx, s0, s1, s2, s3]() { return sy_sppf_pool(ctx, s0, s1, s2, s3); }, {s0, s1, s2, s3});
    conv(s.cv2, buf, out, s.add ? x : nullptr);  // Add(pooled, x), fused
  }
  // C2PSA (PtModel.cs:339) with PSABlock (:341) and Attention (:429-437):
  //   b1 = b + proj(attn_o + pe(v)),  b = b1 + f1(f0(b1)).
  void c2psa(const C2psaM& p, sy_tensor* x, sy_tensor* out) {
    const int c = p.c;
    sy_tensor* buf = alloc(x->n, 2 * c, x->h, x->w);
    conv(p.cv1, x, buf);
    sy_tensor* b = slice(buf, c, c);
    for (const PsaM& blk : p.m) psa_block(blk, b, b);  // back into the b slice
    conv(p.cv2, buf, out);
  }
  // PSABlock (PtModel.cs:341) with Attention (:429-437), residuals fused:
  //   b1 = x + proj(attn_o + pe(v)),  out = b1 + f1(f0(b1)).
  // `out` may be `x` (every read of x precedes the last conv).
  void psa_block(const PsaM& blk, sy_tensor* x, sy_tensor* out) {
    const int c = x->c;
    sy_ctx* ctx = m->ctx;
    sy_tensor* qkv = alloc(x->n, blk.qkv.oc, x->h, x->w);
    conv(blk.qkv, x, qkv);
    sy_tensor* o = alloc(x->n, c, x->h, x->w);
    sy_tensor* v = alloc(x->n, c, x->h, x->w);
    const int heads = blk.heads, kd = blk.kd, hd = blk.hd;
    const float scale = blk.scale;
    op([ctx, qkv, heads, kd, hd, scale, o, v]() { return sy_attention(ctx, qkv, heads, kd, hd, scale, o, v); },
       {qkv, o, v});
    reserve(attention_scratch_bytes(x->n, x->h, x->w, heads, hd));
    sy_tensor* s = alloc(x->n, c, x->h, x->w);
    conv(blk.pe, v, s, o);  // attended + pe(v)
    sy_tensor* b1 = alloc(x->n, c, x->h, x->w);
    conv(blk.proj, s, b1, x);  // x + attn(x)
    sy_tensor* f = alloc(x->n, 2 * c, x->h, x->w);
    conv(blk.f0, b1, f);
    conv(blk.f1, f, out, b1);  // b1 + ffn(b1)
  }
  void upsample(sy_tensor* x, sy_tensor* out) {
    sy_ctx* ctx = m->ctx;
    op([ctx, x, out]() { return sy_resize_nearest(ctx, x, out); }, {x, out});
  }
  // Detect level: box chain into R[0:4*reg], class chain into R[4*reg:].
  // Segment: the mask-coefficient branch writes R[4*reg + nc:], which the
  // decode appends to the head.
  sy_tensor* detect_level(const DetectM& d, sy_tensor* f, int reg, int nc, const SegM* sg = nullptr, int lvl = 0) {
    const int B = f->n;
    const int nm = sg ? sg->nm : 0;
    sy_tensor* r = alloc(B, 4 * reg + nc + nm, f->h, f->w);
    sy_tensor* box_out = slice(r, 0, 4 * reg);
    sy_tensor* cls_out = slice(r, 4 * reg, nc);
    if (sg) {
      sy_tensor* m0 = conv_new(sg->cv4[lvl][0], f);
      sy_tensor* m1 = conv_new(sg->cv4[lvl][1], m0);
      conv(sg->cv4[lvl][2], m1, slice(r, 4 * reg + nc, nm));
    }
    if (d.fused_first) {
      const int c2 = d.box_ch, c3 = d.cls_ch;
      sy_tensor* a = alloc(B, c2 + c3, f->h, f->w);
      conv(d.first, f, a);
      sy_tensor* b = alloc(B, c2 + c3, f->h, f->w);
      conv(d.box[0], slice(a, 0, c2), slice(b, 0, c2));
      conv(d.cls[0], slice(a, c2, c3), slice(b, c2, c3));
      conv(d.box[1], slice(b, 0, c2), box_out);
      conv(d.cls[1], slice(b, c2, c3), cls_out);
      return r;
    }
    auto chain = [&](const std::vector<Conv>& cs, sy_tensor* in, sy_tensor* dst) {
      sy_tensor* cur = in;
      for (size_t i = 0; i < cs.size(); ++i) {
        if (i + 1 == cs.size()) {
          conv(cs[i], cur, dst);
        } else {
          cur = conv_new(cs[i], cur);
        }
      }
    };
    chain(d.box, f, box_out);
    chain(d.cls, f, cls_out);
    return r;
  }

  // Proto on the P3 feature; its NHWC result is laid out NCHW into `dst`.
  void proto(const SegM& sg, sy_tensor* f, float** dst_slot) {
    sy_tensor* a = conv_new(sg.p_cv1, f);
    sy_tensor* u = alloc(f->n, sg.npr, 2 * f->h, 2 * f->w);
    conv(sg.p_up, a, u);
    sy_tensor* b = conv_new(sg.p_cv2, u);
    sy_tensor* pr = conv_new(sg.p_cv3, b);
    sy_ctx* ctx = m->ctx;
    op([ctx, pr, dst_slot]() { return op_view_to_nchw(ctx, pr, *dst_slot); }, {pr});
  }
  // Proto26 (PtModel.cs:345-352): r = f0 + up2(refine0(f1)) + up4(refine1(f2))
  // in the reference's order, then feat_fuse and Proto.
  void proto26(const SegM& sg, sy_tensor* f0, sy_tensor* f1, sy_tensor* f2, float** dst_slot) {
    sy_ctx* ctx = m->ctx;
    sy_tensor* hi[2] = {conv_new(sg.refine[0], f1), conv_new(sg.refine[1], f2)};
    sy_tensor* r = f0;
    for (int i = 0; i < 2; ++i) {
      sy_tensor* up = alloc(f0->n, f0->c, f0->h, f0->w);
      sy_tensor* h = hi[i];
      op([ctx, h, up]() { return sy_resize_nearest(ctx, h, up); }, {h, up});
      sy_tensor* sum = alloc(f0->n, f0->c, f0->h, f0->w);
      sy_tensor* a = r;
      op([ctx, a, up, sum]() { return sy_add(ctx, a, up, sum); }, {a, up, sum});
      r = sum;
    }
    proto(sg, conv_new(sg.fuse, r), dst_slot);
  }

  void resolve(char* base) {
    for (auto& fx : fixed) fx.first->data = (float*)(base + fx.second);
    for (auto& fx : fixups) fx.first->data = (float*)(base + bufs[fx.second].off);
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
  const std::vector<Layer>& ls = m->layers;
  const int n = (int)ls.size();
  // Spatial size of every layer's output (PtModel.Run routing).
  std::vector<int> hh(n), ww(n);
  auto in_hw = [&](int f, int* h, int* w) {
    if (f < 0) { *h = H; *w = W; } else { *h = hh[f]; *w = ww[f]; }
  };
  for (int i = 0; i < n; ++i) {
    int h0, w0;
    in_hw(ls[i].from[0], &h0, &w0);
    if (ls[i].type == L_CONV) {
      const int hi = h0, wi = w0;
      SY_TRY(sy_conv_out_size(m->ctx, ls[i].conv.id, hi, wi, &h0, &w0));
    } else if (ls[i].type == L_UP) {
      h0 *= 2;
      w0 *= 2;
    }
    hh[i] = h0;
    ww[i] = w0;
  }
  const int anchors = (H / 8) * (W / 8) + (H / 16) * (W / 16) + (H / 32) * (W / 32);
  // Input and output live in the plan arena too.
  p.used = (size_t)B * 3 * H * W * sizeof(float);
  p.used = (p.used + 255) & ~size_t(255);
  const int nm = m->cfg.nm > 0 ? m->cfg.nm : 0;
  const bool e2e = end_to_end(m->cfg);
  const int kept = anchors < kEndToEndMaxDet ? anchors : kEndToEndMaxDet;
  const size_t head_off = p.used;
  p.used += (size_t)B * (nc + 4 + nm) * anchors * sizeof(float);
  p.used = (p.used + 255) & ~size_t(255);
  const size_t out_off = e2e ? p.used : head_off;
  if (e2e) p.used += (size_t)B * kept * (6 + nm) * sizeof(float);
  p.used = (p.used + 255) & ~size_t(255);
  const size_t proto_off = p.used;
  if (nm) p.used += (size_t)B * nm * (H / 4) * (W / 4) * sizeof(float);
  auto input = std::make_unique<sy_tensor>(sy_tensor{nullptr, B, 3, H, W, 3, SY_LAYOUT_NCHW});
  p.fixed.emplace_back(input.get(), 0);
  sy_tensor* x = input.get();
  p.store.push_back(std::move(input));

  // Concat buffers first; their inputs write in place.
  std::vector<sy_tensor*> out(n, nullptr);
  std::vector<sy_tensor*> dest(n, nullptr);
  for (int i = 0; i < n; ++i) {
    if (ls[i].type != L_CAT) continue;
    sy_tensor* buf = p.alloc(B, ls[i].c, hh[i], ww[i]);
    out[i] = buf;
    int c0 = 0;
    for (int f : ls[i].from) {
      const int cf = f < 0 ? 3 : ls[f].c;
      if (f >= 0 && ls[f].type != L_CAT && ls[f].type != L_DETECT && !dest[f]) dest[f] = p.slice(buf, c0, cf);
      c0 += cf;
    }
  }
  auto input_of = [&](int f) { return f < 0 ? x : out[f]; };
  // A 2x upsample whose only reader is the leading slice of a concat read
  // only by a C2f is not materialised: the C2f's 1x1 cv1 reads those
  // channels from the upsample's half-resolution source (fused_up[concat] =
  // the upsample layer).
  std::vector<int> fused_up(n, -1);
  for (int j = 0; j < n; ++j) {
    if (ls[j].type != L_CAT || ls[j].from.empty()) continue;
    const int u = ls[j].from[0];
    if (u < 0 || ls[u].type != L_UP || !dest[u] || ls[u].from.empty() || ls[u].from[0] < 0) continue;
    const int s = ls[u].from[0];
    if (hh[u] != 2 * hh[s] || ww[u] != 2 * ww[s] || ls[u].c % 32 != 0) continue;
    int readers_j = 0, readers_u = 0, c2f_reader = -1;
    for (int k = 0; k < n; ++k)
      for (int f : ls[k].from) {
        if (f == j) {
          ++readers_j;
          if (ls[k].type == L_C2F && ls[k].from[0] == j) c2f_reader = k;
        }
        if (f == u) ++readers_u;
      }
    if (readers_j == 1 && c2f_reader >= 0 && readers_u == 1) fused_up[j] = u;
  }
  auto is_fused_up = [&](int u) {
    for (int j = 0; j < n; ++j)
      if (fused_up[j] == u) return true;
    return false;
  };
  // The stride-8 detect level (and the Segment prototypes) depend only on the
  // P3 feature, the stride-16 level only on P4: as branches they can run
  // beside the rest of the neck, whose 40x40 and 20x20 layers leave much of
  // the GPU idle.  Level 1 branches off P3's head, level 2 also P4's.
  int branch_from[2] = {-1, -1};
  for (int i = 0; i < n; ++i)
    if (ls[i].type == L_DETECT) {
      branch_from[0] = ls[i].from[0];
      branch_from[1] = ls[i].from[1];
    }
  std::vector<sy_tensor*> levels;
  for (int i = 0; i < n; ++i) {
    const Layer& l = ls[i];
    sy_tensor* src = input_of(l.from[0]);
    sy_tensor* dst = dest[i];
    auto own = [&]() { return dst ? dst : p.alloc(B, l.c, hh[i], ww[i]); };
    switch (l.type) {
      case L_CONV: out[i] = own(); p.conv(l.conv, src, out[i]); break;
      case L_C2F: {
        out[i] = own();
        const int u = l.from[0] >= 0 ? fused_up[l.from[0]] : -1;
        p.c2f(l.c2f, src, out[i], u >= 0 ? input_of(ls[u].from[0]) : nullptr);
        break;
      }
      case L_SPPF: out[i] = own(); p.sppf(l.sppf, src, out[i]); break;
      case L_C2PSA: out[i] = own(); p.c2psa(l.psa, src, out[i]); break;
      case L_UP:
        out[i] = own();
        if (!is_fused_up(i)) p.upsample(src, out[i]);
        break;
      case L_CAT: {
        // Inputs not written in place (none in these topologies) are copied.
        int c0 = 0;
        for (int f : l.from) {
          const int cf = f < 0 ? 3 : ls[f].c;
          sy_tensor* slot = p.slice(out[i], c0, cf);
          if (f < 0 || !dest[f] || dest[f] != out[f]) {
            sy_tensor* from = input_of(f);
            sy_ctx* ctx = m->ctx;
            p.op([ctx, from, slot]() { return sy_copy(ctx, from, slot); }, {from, slot});
          }
          c0 += cf;
        }
        break;
      }
      case L_DETECT:
        for (int j = 0; j < 3; ++j) {
          p.lane = j < 2 && l.from[j] == branch_from[j] ? j + 1 : 0;
          levels.push_back(p.detect_level(l.det[j], input_of(l.from[j]), reg, nc, nm ? &l.seg : nullptr, j));
          if (j == 0 && nm && !l.seg.proto26) p.proto(l.seg, input_of(l.from[0]), &plan->proto);
        }
        p.lane = 0;
        p.join();
        // Proto26 reads all three levels: on the main chain after the join.
        if (nm && l.seg.proto26)
          p.proto26(l.seg, input_of(l.from[0]), input_of(l.from[1]), input_of(l.from[2]), &plan->proto);
        break;
    }
    for (int k = 0; k < 2; ++k)
      if (i == branch_from[k]) p.fork(k + 1);
  }
  {
    sy_ctx* ctx = m->ctx;
    Plan* pl = plan;
    const int total = anchors;
    auto lv = std::make_shared<std::vector<sy_tensor*>>(levels);
    // End-to-end heads decode to x1 y1 x2 y2 (PtModel.cs:449-504 passes
    // xyxy = end2end) and select with the mask coefficients as extras
    // (CompleteInstanceHead, PtModel.cs:506-523; EndToEndTopK, :530-570).
    const int xyxy = e2e ? 1 : 0;
    p.op(
        [ctx, pl, lv, total, nc, reg, xyxy]() {
          sy_tensor t[3] = {*(*lv)[0], *(*lv)[1], *(*lv)[2]};
          const float strides[3] = {8.f, 16.f, 32.f};
          return sy_detect_decode(ctx, t, strides, 3, reg, nc, xyxy, pl->head, total);
        },
        {levels[0], levels[1], levels[2]});
    if (e2e) {
      const int channels = nc + 4 + nm;
      p.op([ctx, pl, B, channels, total, nc]() {
        return sy_e2e_topk(ctx, pl->head, B, channels, total, nc, kEndToEndMaxDet, 0, pl->output);
      }, {});
      size_t need = 0;
      SY_TRY(e2e_topk_scratch_bytes(B, channels, total, nc, kEndToEndMaxDet, &need));
      p.reserve(need);
    }
  }
  plan->unshared_bytes = p.used + p.unshared();
  plan->bytes = p.pack(p.used);
  SY_HIP(hipMalloc((void**)&plan->arena, plan->bytes));
  p.resolve(plan->arena);
  plan->input = (float*)plan->arena;
  plan->head = (float*)(plan->arena + head_off);
  plan->output = (float*)(plan->arena + out_off);
  if (nm) plan->proto = (float*)(plan->arena + proto_off);
  // Keep the views alive for the lifetime of the ops.
  auto keep = std::make_shared<std::vector<std::unique_ptr<sy_tensor>>>(std::move(p.store));
  plan->ops.push_back(Plan::Op{Plan::kOp, 0, [keep]() { return SY_OK; }});
  SY_TRY(ensure_scratch(m->ctx, plan->scratch));
  for (hipEvent_t& e : plan->fork_ev) SY_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
  SY_HIP(hipEventCreateWithFlags(&plan->join_ev, hipEventDisableTiming));
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

// level L > 0: ops of lanes 1..L on the side stream, forked from and joined
// back to the main stream by events (only while capturing the plan's graph).
int run_ops(sy_ctx* ctx, Plan* plan, int level) {
  bool forked = false;
  bool recorded[Plan::kMaxLevel] = {false, false};
  bool pending[Plan::kMaxLevel] = {false, false};  // fork recorded, not yet waited on
  for (auto& op : plan->ops) {
    if (op.kind == Plan::kFork) {
      if (op.lane <= level) {
        if (!ctx->side) SY_HIP(hipStreamCreateWithFlags(&ctx->side, hipStreamNonBlocking));
        SY_HIP(hipEventRecord(plan->fork_ev[op.lane - 1], ctx->stream));
        recorded[op.lane - 1] = pending[op.lane - 1] = true;
        forked = true;
      }
    } else if (op.kind == Plan::kJoin) {
      if (forked) {
        SY_HIP(hipEventRecord(plan->join_ev, ctx->side));
        SY_HIP(hipStreamWaitEvent(ctx->stream, plan->join_ev, 0));
      }
    } else if (forked && op.lane >= 1 && op.lane <= level) {
      // The side stream waits for its fork only before the branch's first op,
      // so an earlier branch queued on it does not wait for a later fork.
      SY_CHECK(recorded[op.lane - 1], SY_ESTATE, "branch op before its fork");
      if (pending[op.lane - 1]) {
        SY_HIP(hipStreamWaitEvent(ctx->side, plan->fork_ev[op.lane - 1], 0));
        pending[op.lane - 1] = false;
      }
      SideLane side(ctx, true);
      SY_CHECK(side.ok(), SY_EDEVICE, "side stream creation failed");
      SY_TRY(op.f());
    } else {
      SY_TRY(op.f());
    }
  }
  return SY_OK;
}

int capture(sy_ctx* ctx, Plan* plan, int level, uint64_t* g) {
  SY_TRY(sy_graph_begin(ctx));
  int rc = run_ops(ctx, plan, level);
  int rc2 = sy_graph_end(ctx, g);
  SY_TRY(rc);
  return rc2;
}

// Average of `reps` replays of graph g after one warm replay, in ms.
int time_graph(sy_ctx* ctx, uint64_t g, int reps, float* ms) {
  hipEvent_t e0 = nullptr, e1 = nullptr;
  int rc = SY_OK;
  if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) rc = SY_EDEVICE;
  if (rc == SY_OK) rc = sy_graph_launch(ctx, g);
  if (rc == SY_OK && hipEventRecord(e0, ctx->stream) != hipSuccess) rc = SY_EDEVICE;
  for (int i = 0; rc == SY_OK && i < reps; ++i) rc = sy_graph_launch(ctx, g);
  if (rc == SY_OK && (hipEventRecord(e1, ctx->stream) != hipSuccess || hipEventSynchronize(e1) != hipSuccess ||
                      hipEventElapsedTime(ms, e0, e1) != hipSuccess))
    rc = SY_EDEVICE;
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (rc == SY_EDEVICE) set_error("timing a captured forward failed");
  if (rc == SY_OK) *ms /= reps;
  return rc;
}

// The forward as one chain on the main stream: eager while profiling or with
// graphs off, else the plan's single-stream graph (captured on first use,
// after the eager tuning pass).
int run_plan_chain(sy_model* m, Plan* plan) {
  sy_ctx* ctx = m->ctx;
  if (!m->use_graph || ctx->profiling) return run_ops(ctx, plan, 0);
  if (plan->graph0 && graph_stale(ctx, plan->graph0)) {
    SY_TRY(sy_graph_destroy(ctx, plan->graph0));
    plan->graph0 = 0;
  }
  if (!plan->warmed) {
    SY_TRY(run_ops(ctx, plan, 0));
    SY_HIP(hipStreamSynchronize(ctx->stream));
    plan->warmed = true;
    plan->level = m->branch_level;  // run_plan still picks its branch level by timing
  }
  if (!plan->graph0) {
    SY_TRY(ensure_scratch(ctx, plan->scratch));
    SY_TRY(capture(ctx, plan, 0, &plan->graph0));
  }
  return sy_graph_launch(ctx, plan->graph0);
}

int run_plan(sy_model* m, Plan* plan) {
  sy_ctx* ctx = m->ctx;
  if (!m->use_graph || ctx->profiling) return run_ops(ctx, plan, 0);
  if (plan->graph && graph_stale(ctx, plan->graph)) {
    // Another plan grew the shared scratch buffer: capture again.
    SY_TRY(sy_graph_destroy(ctx, plan->graph));
    plan->graph = 0;
  }
  if (!plan->warmed) {
    // One eager pass first: convolutions tune their algorithm and tile for
    // these shapes (timed on the device) before anything is captured.
    SY_TRY(run_ops(ctx, plan, 0));
    SY_HIP(hipStreamSynchronize(ctx->stream));
    plan->warmed = true;
    plan->level = m->branch_level;
  }
  if (!plan->graph) {
    // The branch ops run on the side stream with its own scratch buffer,
    // which must not grow during capture.
    {
      SideLane side(ctx, true);
      SY_CHECK(side.ok(), SY_EDEVICE, "side stream creation failed");
      SY_TRY(ensure_scratch(ctx, plan->scratch));
    }
    if (plan->level >= 0) {
      // Recapture (the scratch moved) with the level chosen before.
      SY_TRY(capture(ctx, plan, plan->level, &plan->graph));
    } else {
      // Capture the forward once per branch level and keep the fastest: the
      // branches pay off when the neck's small layers leave the GPU idle
      // (large batches), not when every layer is latency-bound (batch 1).
      // Ops must not allocate during capture (scratch was reserved).
      uint64_t best = 0;
      float best_ms = 0.f;
      for (int level = 0; level <= Plan::kMaxLevel; ++level) {
        uint64_t g = 0;
        SY_TRY(capture(ctx, plan, level, &g));
        float ms = 0.f;
        int rc = time_graph(ctx, g, 3, &ms);
        if (rc != SY_OK) {
          (void)sy_graph_destroy(ctx, g);
          if (best) (void)sy_graph_destroy(ctx, best);
          return rc;
        }
        if (!best || ms < best_ms) {
          if (best) SY_TRY(sy_graph_destroy(ctx, best));
          best = g;
          best_ms = ms;
          plan->level = level;
        } else {
          SY_TRY(sy_graph_destroy(ctx, g));
        }
      }
      plan->graph = best;
    }
  }
  return sy_graph_launch(ctx, plan->graph);
}

int ensure_host_io(sy_model* m, size_t in_bytes, size_t out_bytes) {
  SY_CHECK(!m->ctx->capturing, SY_ESTATE, "host I/O staging during graph capture");
  if (!m->io) {
    auto io = std::make_unique<HostIO>();
    // Streams at the default priority, like every stream of the library.
    SY_HIP(hipStreamCreateWithFlags(&io->up, hipStreamNonBlocking));
    SY_HIP(hipStreamCreateWithFlags(&io->down, hipStreamNonBlocking));
    for (int i = 0; i < HostIO::kSlots; ++i) {
      SY_HIP(hipHostMalloc((void**)&io->pin_in[i], HostIO::kPiece, hipHostMallocDefault));
      SY_HIP(hipHostMalloc((void**)&io->pin_out[i], HostIO::kPiece, hipHostMallocDefault));
      SY_HIP(hipEventCreateWithFlags(&io->in_slot[i], hipEventDisableTiming));
      SY_HIP(hipEventCreateWithFlags(&io->out_slot[i], hipEventDisableTiming));
    }
    for (int i = 0; i < 2; ++i)
      for (hipEvent_t* e : {&io->in_ready[i], &io->in_free[i], &io->out_ready[i], &io->out_free[i]})
        SY_HIP(hipEventCreateWithFlags(e, hipEventDisableTiming));
    // Two copiers: four threads (one the caller) fill pinned memory at
    // ~75 GB/s, above the ~57 GB/s of PCIe DMA; six empty it into the
    // caller's output, which is usually freshly allocated and pays a page
    // fault per page on first write.
    const unsigned hw = std::thread::hardware_concurrency();
    io->pool = std::make_unique<CopyPool>((int)std::min(3u, hw > 4 ? hw / 4 : 0u));
    io->pool_down = std::make_unique<CopyPool>((int)std::min(5u, hw > 4 ? hw / 3 : 0u));
    m->io = std::move(io);
  }
  HostIO& io = *m->io;
  if (io.dev_in_bytes < in_bytes || io.dev_out_bytes < out_bytes) {
    SY_HIP(hipStreamSynchronize(m->ctx->stream));
    SY_HIP(hipStreamSynchronize(io.up));
    SY_HIP(hipStreamSynchronize(io.down));
    for (int i = 0; i < 2; ++i) {
      if (io.dev_in_bytes < in_bytes) {
        if (io.dev_in[i]) SY_HIP(hipFree(io.dev_in[i]));
        io.dev_in[i] = nullptr;
        SY_HIP(hipMalloc((void**)&io.dev_in[i], in_bytes));
      }
      if (io.dev_out_bytes < out_bytes) {
        if (io.dev_out[i]) SY_HIP(hipFree(io.dev_out[i]));
        io.dev_out[i] = nullptr;
        SY_HIP(hipMalloc((void**)&io.dev_out[i], out_bytes));
      }
    }
    io.dev_in_bytes = std::max(io.dev_in_bytes, in_bytes);
    io.dev_out_bytes = std::max(io.dev_out_bytes, out_bytes);
  }
  return SY_OK;
}

// sy_model_predict_raw / _seg from pageable host buffers.  Batches of 8 or
// more images run as four chunks (a plan for the chunk size) in a pipeline:
// while chunk i runs its forward, chunk i + 1 goes up and chunk i - 1 comes
// down, each over PCIe from pinned staging that host threads fill or empty
// in 8 MiB pieces.  Device buffers for two chunks in flight decouple the
// copies from the plan's own input and output, which every chunk's forward
// reuses.  Smaller batches are one chunk (its pieces still overlap the host
// copies with the DMA).
int predict_host(sy_model* m, const float* input, int B, int H, int W, float* out, float* proto_out) {
  sy_ctx* ctx = m->ctx;
  SY_CHECK(!ctx->capturing, SY_ESTATE, "host I/O during graph capture");
  int ch_out = 0, an_out = 0;
  SY_TRY(sy_model_output_shape(m, B, H, W, &ch_out, &an_out));
  const int nm = m->cfg.nm > 0 ? m->cfg.nm : 0;
  const size_t in_img = (size_t)3 * H * W * sizeof(float);
  const size_t out_img = (size_t)ch_out * an_out * sizeof(float);
  const size_t proto_img = proto_out ? (size_t)nm * (H / 4) * (W / 4) * sizeof(float) : 0;
  // Chunks per call (SIMDYOLO_HIP_IO_CHUNKS overrides): more chunks overlap
  // more of the PCIe time, fewer keep the forward's batch efficiency.
  int nchunks = B >= 16 ? 2 : 1;
  if (const char* e = getenv("SIMDYOLO_HIP_IO_CHUNKS")) nchunks = std::max(1, std::min(B, atoi(e)));
  const int chunk = (B + nchunks - 1) / nchunks;
  SY_TRY(ensure_host_io(m, (size_t)chunk * in_img, (size_t)chunk * (out_img + proto_img)));
  HostIO& io = *m->io;
  struct Chunk {
    int i0, n;
    Plan* plan;
  };
  std::vector<Chunk> chunks;
  for (int i0 = 0; i0 < B; i0 += chunk) {
    Chunk c{i0, std::min(chunk, B - i0), nullptr};
    SY_TRY(get_plan(m, c.n, H, W, &c.plan));
    chunks.push_back(c);
  }
  int in_next = 0, out_next = 0;
  // Chunk k's input into `dst` (a staging buffer, or the plan's own input
  // when there is one chunk).
  auto upload = [&](size_t k, char* dst) -> int {
    const Chunk& c = chunks[k];
    const int s = (int)(k & 1);
    if (dst == io.dev_in[s] && io.in_free_rec[s]) SY_HIP(hipStreamWaitEvent(io.up, io.in_free[s], 0));
    const char* src = (const char*)input + (size_t)c.i0 * in_img;
    const size_t total = (size_t)c.n * in_img;
    for (size_t off = 0; off < total; off += HostIO::kPiece) {
      const size_t len = std::min(HostIO::kPiece, total - off);
      const int slot = in_next;
      in_next = (in_next + 1) % HostIO::kSlots;
      if (io.in_slot_used[slot]) SY_HIP(hipEventSynchronize(io.in_slot[slot]));
      io.pool->copy(io.pin_in[slot], src + off, len);
      SY_HIP(hipMemcpyAsync(dst + off, io.pin_in[slot], len, hipMemcpyHostToDevice, io.up));
      SY_HIP(hipEventRecord(io.in_slot[slot], io.up));
      io.in_slot_used[slot] = true;
    }
    SY_HIP(hipEventRecord(io.in_ready[s], io.up));
    return SY_OK;
  };
  auto forward = [&](size_t k) -> int {
    const Chunk& c = chunks[k];
    const int s = (int)(k & 1);
    SY_HIP(hipStreamWaitEvent(ctx->stream, io.in_ready[s], 0));
    SY_HIP(hipMemcpyAsync(c.plan->input, io.dev_in[s], (size_t)c.n * in_img, hipMemcpyDeviceToDevice, ctx->stream));
    SY_HIP(hipEventRecord(io.in_free[s], ctx->stream));
    io.in_free_rec[s] = true;
    SY_TRY(run_plan_chain(m, c.plan));
    if (io.out_free_rec[s]) SY_HIP(hipStreamWaitEvent(ctx->stream, io.out_free[s], 0));
    SY_HIP(hipMemcpyAsync(io.dev_out[s], c.plan->output, (size_t)c.n * out_img, hipMemcpyDeviceToDevice,
                          ctx->stream));
    if (proto_img)
      SY_HIP(hipMemcpyAsync(io.dev_out[s] + (size_t)c.n * out_img, c.plan->proto, (size_t)c.n * proto_img,
                            hipMemcpyDeviceToDevice, ctx->stream));
    SY_HIP(hipEventRecord(io.out_ready[s], ctx->stream));
    return SY_OK;
  };
  // Pieces of chunk k's outputs: the head, then the prototypes.  `released`
  // runs once the last D2H of the chunk is enqueued and dev_out's release
  // event recorded behind it (from then on the next forward may reuse it).
  std::function<void(size_t)> released = [](size_t) {};
  // Chunk k's outputs from the staging buffer, or from the plan's own
  // output (and prototype) buffers when `direct`.
  auto download = [&](size_t k, bool direct) -> int {
    const Chunk& c = chunks[k];
    const int s = (int)(k & 1);
    SY_HIP(hipStreamWaitEvent(io.down, io.out_ready[s], 0));
    struct Piece {
      size_t dev_off, len;
      char* dst;
      int slot;
    };
    std::vector<Piece> pieces;
    std::vector<const char*> bases;
    auto add = [&](const char* src, size_t total, char* dst) {
      for (size_t off = 0; off < total; off += HostIO::kPiece) {
        pieces.push_back(Piece{off, std::min(HostIO::kPiece, total - off), dst + off, -1});
        bases.push_back(src);
      }
    };
    const char* head_src = direct ? (const char*)c.plan->output : io.dev_out[s];
    const char* proto_src = direct ? (const char*)c.plan->proto : io.dev_out[s] + (size_t)c.n * out_img;
    add(head_src, (size_t)c.n * out_img, (char*)out + (size_t)c.i0 * out_img);
    if (proto_img) add(proto_src, (size_t)c.n * proto_img, (char*)proto_out + (size_t)c.i0 * proto_img);

    // Up to kSlots pieces in flight; the host empties them in order.
    size_t issued = 0;
    for (size_t done = 0; done < pieces.size(); ++done) {
      while (issued < pieces.size() && issued < done + HostIO::kSlots) {
        const char* base = bases[issued];
        Piece& p = pieces[issued++];
        p.slot = out_next;
        out_next = (out_next + 1) % HostIO::kSlots;
        SY_HIP(hipMemcpyAsync(io.pin_out[p.slot], base + p.dev_off, p.len, hipMemcpyDeviceToHost, io.down));
        SY_HIP(hipEventRecord(io.out_slot[p.slot], io.down));
        if (issued == pieces.size() && !direct) {
          SY_HIP(hipEventRecord(io.out_free[s], io.down));
          io.out_free_rec[s] = true;
          released(k);
        }
      }
      if (done == 0) {
        // The first pieces are queued behind the forward: meanwhile fault in
        // the caller's output pages.
        io.pool_down->touch((char*)out + (size_t)c.i0 * out_img, (size_t)c.n * out_img);
        if (proto_img) io.pool_down->touch((char*)proto_out + (size_t)c.i0 * proto_img, (size_t)c.n * proto_img);
      }
      const Piece& p = pieces[done];
      SY_HIP(hipEventSynchronize(io.out_slot[p.slot]));
      io.pool_down->copy(p.dst, io.pin_out[p.slot], p.len);
    }
    return SY_OK;
  };
  if (chunks.size() == 1) {
    // One chunk: nothing to overlap with the forward, so the copies go
    // straight to and from the plan's buffers (the previous call has
    // finished with them) and the forward runs the plan's timed, possibly
    // branched, graph.
    const Chunk& c = chunks[0];
    SY_TRY(upload(0, (char*)c.plan->input));
    SY_HIP(hipStreamWaitEvent(ctx->stream, io.in_ready[0], 0));
    SY_TRY(run_plan(m, c.plan));
    SY_HIP(hipEventRecord(io.out_ready[0], ctx->stream));
    SY_TRY(download(0, true));
  } else {
    // This thread uploads chunk after chunk and enqueues each forward; a
    // second thread downloads each chunk once its forward is enqueued.
    std::mutex mu;
    std::condition_variable cv;
    size_t enqueued = 0;  // forwards enqueued
    size_t freed = 0;     // chunks whose dev_out release is recorded
    bool failed = false;
    released = [&](size_t k) {
      std::lock_guard<std::mutex> lock(mu);
      freed = k + 1;
      cv.notify_all();
    };
    int down_rc = SY_OK;
    std::string down_err;
    std::thread downloader([&] {
      for (size_t k = 0; k < chunks.size(); ++k) {
        {
          std::unique_lock<std::mutex> lock(mu);
          cv.wait(lock, [&] { return enqueued > k || failed; });
          if (enqueued <= k) return;  // the uploader stopped
        }
        const int rc = download(k, false);
        if (rc != SY_OK) {
          std::lock_guard<std::mutex> lock(mu);
          down_rc = rc;
          down_err = sy_last_error();
          failed = true;
          cv.notify_all();
          return;
        }
      }
    });
    int rc = SY_OK;
    for (size_t k = 0; k < chunks.size() && rc == SY_OK; ++k) {
      rc = upload(k, io.dev_in[k & 1]);
      if (rc == SY_OK && k >= 2) {
        // Chunk k's forward writes dev_out[k % 2]: chunk k - 2's downloads
        // must be enqueued (and its release recorded) first.
        std::unique_lock<std::mutex> lock(mu);
        cv.wait(lock, [&] { return freed >= k - 1 || failed; });
        if (freed < k - 1) rc = SY_EDEVICE;  // the downloader failed; its error is reported below
      }
      if (rc == SY_OK) rc = forward(k);
      std::lock_guard<std::mutex> lock(mu);
      if (rc == SY_OK) ++enqueued; else failed = true;
      cv.notify_all();
    }
    downloader.join();
    if (down_rc != SY_OK) {
      set_error("%s", down_err.c_str());
      return down_rc;
    }
    if (rc != SY_OK) return rc;
  }
  SY_HIP(hipStreamSynchronize(io.down));
  SY_HIP(hipStreamSynchronize(io.up));
  SY_HIP(hipStreamSynchronize(ctx->stream));
  return prof_collect(ctx);
}

}  // namespace

extern "C" {

int sy_model_layout(const sy_model_config* cfg, int32_t* out, int max_entries, int* count) {
  SY_TRY(validate_cfg(cfg));
  SY_CHECK(count, SY_EINVAL, "null count");
  Builder b{nullptr, {}, false};
  b.pw.layout = out;
  b.pw.max_entries = out ? max_entries : 0;
  b.pw.eps = cfg->bn_eps;
  std::vector<Layer> ls;
  build_layers(b, *cfg, ls);
  *count = b.pw.count;
  return SY_OK;
}

int sy_model_create(sy_ctx* ctx, const sy_model_config* cfg, const float* params, size_t n_params, sy_model** out) {
  SY_CHECK(ctx && params && out, SY_EINVAL, "null argument");
  SY_TRY(validate_cfg(cfg));
  *out = nullptr;
  {
    // Size check before any device work.
    Builder probe{nullptr, {}, false};
    probe.pw.eps = cfg->bn_eps;
    std::vector<Layer> ls;
    build_layers(probe, *cfg, ls);
    SY_CHECK(probe.pw.pos == n_params, SY_EINVAL, "parameter blob holds %zu floats, the model needs %zu", n_params,
             probe.pw.pos);
  }
  auto m = std::make_unique<sy_model>();
  m->ctx = ctx;
  m->cfg = *cfg;
  Builder b{m.get(), {}, true};
  b.ctx = ctx;
  b.pw.params = params;
  b.pw.n_params = n_params;
  b.pw.eps = cfg->bn_eps;
  build_layers(b, *cfg, m->layers);
  SY_TRY(b.rc);
  SY_CHECK(!b.pw.overrun && b.pw.pos == n_params, SY_EINVAL, "parameter blob size mismatch");
  m->weight_bytes = b.weight_bytes;
  *out = m.release();
  return SY_OK;
}

void sy_model_destroy(sy_model* model) { delete model; }

int sy_model_output_shape(sy_model* m, int batch, int h, int w, int* channels, int* anchors) {
  SY_CHECK(m && channels && anchors, SY_EINVAL, "null argument");
  SY_CHECK(batch > 0 && h > 0 && w > 0 && h % 32 == 0 && w % 32 == 0, SY_EINVAL, "invalid input shape");
  const int nm = m->cfg.nm > 0 ? m->cfg.nm : 0;
  const int total = (h / 8) * (w / 8) + (h / 16) * (w / 16) + (h / 32) * (w / 32);
  if (end_to_end(m->cfg)) {
    *channels = total < kEndToEndMaxDet ? total : kEndToEndMaxDet;
    *anchors = 6 + nm;
  } else {
    *channels = m->cfg.nc + 4 + nm;
    *anchors = total;
  }
  return SY_OK;
}

int sy_model_head(sy_model* m, int batch, int h, int w, float** head, int* channels, int* anchors) {
  SY_CHECK(m, SY_EINVAL, "null model");
  Plan* plan = nullptr;
  SY_TRY(get_plan(m, batch, h, w, &plan));
  if (head) *head = plan->head;
  if (channels) *channels = m->cfg.nc + 4 + (m->cfg.nm > 0 ? m->cfg.nm : 0);
  if (anchors) *anchors = (h / 8) * (w / 8) + (h / 16) * (w / 16) + (h / 32) * (w / 32);
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
  SY_CHECK(batch > 0 && h > 0 && w > 0 && h % 32 == 0 && w % 32 == 0, SY_EINVAL,
           "PT YOLO expects NCHW RGB with height/width multiples of 32 (got %dx%d)", h, w);
  return predict_host(m, input, batch, h, w, out, nullptr);
}

int sy_model_proto(sy_model* m, int batch, int h, int w, float** proto, int* channels, int* proto_h, int* proto_w) {
  SY_CHECK(m, SY_EINVAL, "null model");
  SY_CHECK(m->cfg.nm > 0, SY_EINVAL, "the model has no Segment head");
  Plan* plan = nullptr;
  SY_TRY(get_plan(m, batch, h, w, &plan));
  if (proto) *proto = plan->proto;
  if (channels) *channels = m->cfg.nm;
  if (proto_h) *proto_h = h / 4;
  if (proto_w) *proto_w = w / 4;
  return SY_OK;
}

int sy_model_predict_seg(sy_model* m, const float* input, int batch, int h, int w, float* out, float* proto_out) {
  SY_CHECK(m && input && out && proto_out, SY_EINVAL, "null argument");
  SY_CHECK(m->cfg.nm > 0, SY_EINVAL, "the model has no Segment head");
  SY_CHECK(batch > 0 && h > 0 && w > 0 && h % 32 == 0 && w % 32 == 0, SY_EINVAL,
           "PT YOLO expects NCHW RGB with height/width multiples of 32 (got %dx%d)", h, w);
  return predict_host(m, input, batch, h, w, out, proto_out);
}

int sy_model_set_graph(sy_model* m, int use_graph) {
  SY_CHECK(m, SY_EINVAL, "null model");
  m->use_graph = use_graph != 0;
  return SY_OK;
}

int sy_model_set_branch_level(sy_model* m, int level) {
  SY_CHECK(m, SY_EINVAL, "null model");
  SY_CHECK(level >= -1 && level <= Plan::kMaxLevel, SY_EINVAL, "branch level %d out of range -1..%d", level,
           Plan::kMaxLevel);
  SY_CHECK(!m->ctx->capturing, SY_ESTATE, "branch level changed during capture");
  m->branch_level = level;
  for (auto& kv : m->plans) {
    Plan* plan = kv.second.get();
    if (plan->graph) SY_TRY(sy_graph_destroy(m->ctx, plan->graph));
    plan->graph = 0;
    plan->level = level;
  }
  return SY_OK;
}

int sy_model_branch_level(sy_model* m, int batch, int h, int w, int* level) {
  SY_CHECK(m && level, SY_EINVAL, "null argument");
  auto it = m->plans.find(std::make_tuple(batch, h, w));
  *level = (it != m->plans.end() && it->second->graph) ? it->second->level : -1;
  return SY_OK;
}

int sy_model_plan_memory(sy_model* m, int batch, int h, int w, size_t* arena_bytes, size_t* unshared_bytes,
                         size_t* scratch_bytes) {
  SY_CHECK(m, SY_EINVAL, "null model");
  Plan* plan = nullptr;
  SY_TRY(get_plan(m, batch, h, w, &plan));
  if (arena_bytes) *arena_bytes = plan->bytes;
  if (unshared_bytes) *unshared_bytes = plan->unshared_bytes;
  if (scratch_bytes) *scratch_bytes = plan->scratch;
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
