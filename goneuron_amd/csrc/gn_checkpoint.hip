// Checkpoint formats around the device-resident arena (host code).
//
//  - SaveBinaryWeights (net.go:1119-1214) and a reader for it;
//  - SaveGGUF / SaveGGUFExt (net.go:1217-1392, gguf.go): GGUF v3, F32 or F16;
//  - a full training-state file for resume (parameters, Adam moments and
//    timestep, BatchNorm2D running statistics, MoE noise streams).
//
// The tensor list follows the reference: every layer's NamedParams in its
// order (Dense weights [out, in] / biases, Conv2D weights [outC, inC, k, k],
// Embedding / PositionalEncoding weights, TransformerBlock mha_wQ_weights ...
// ff2_biases, RMSNorm gamma, SwiGLU w / v, BatchNorm2D running_mean /
// running_var / gamma / beta), or, for a layer without NamedParams but with
// parameters (SequenceUnroller, MoE), one flat "params" tensor.
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <vector>

#include "gn_common.h"

using namespace gn;

namespace {

struct Tensor {
  std::string name;
  std::vector<int64_t> shape;
  int src = 0;        // 0: parameter arena at off; 1: running mean; 2: running var
  int layer = 0;
  int64_t off = 0, n = 0;
};

// ExtractLayerConfig's type names (net.go:1425-1505); the rest are "Unknown"
const char *layer_type(int kind) {
  switch (kind) {
    case GN_LAYER_DENSE: return "Dense";
    case GN_LAYER_CONV2D: return "Conv2D";
    case GN_LAYER_DROPOUT: return "Dropout";
    case GN_LAYER_MAXPOOL2D: return "MaxPool2D";
    case GN_LAYER_AVGPOOL2D: return "AvgPool2D";
    case GN_LAYER_EMBEDDING: return "Embedding";
    case GN_LAYER_FLATTEN: return "Flatten";
    case GN_LAYER_BATCHNORM2D: return "BatchNorm2D";
    default: return "Unknown";
  }
}

struct Builder {
  std::vector<Tensor> *out;
  int layer;
  int64_t off;
  void add(const std::string &name, std::vector<int64_t> shape) {
    int64_t n = 1;
    for (int64_t d : shape) n *= d;
    Tensor t;
    t.name = name;
    t.shape = std::move(shape);
    t.layer = layer;
    t.off = off;
    t.n = n;
    off += n;
    out->push_back(t);
  }
  void dense(const std::string &pre, int64_t in, int64_t o) {
    add(pre + "weights", {o, in});
    add(pre + "biases", {o});
  }
};

// NamedParams of layer i (names without the file's prefix), parameters at poff
void layer_tensors(gn_model *M, int i, int64_t poff, int64_t pcount, std::vector<Tensor> &v) {
  const gn_layer_desc &d = *model_layer_desc(M, i);
  Builder b{&v, i, poff};
  switch (d.kind) {
    case GN_LAYER_DENSE: b.dense("", d.in_size, d.out_size); return;  // layer.go:860-873
    case GN_LAYER_CONV2D:                                             // conv2d.go:1366-1378
      b.add("weights", {d.out_channels, d.in_channels, d.kernel, d.kernel});
      b.add("biases", {d.out_channels});
      return;
    case GN_LAYER_EMBEDDING: b.add("weights", {d.vocab, d.dim}); return;  // embedding.go:248-256
    case GN_LAYER_POSENC: b.add("weights", {d.seq_len, (int64_t)pcount / d.seq_len}); return;
    case GN_LAYER_RMSNORM: b.add("gamma", {d.dim}); return;  // rmsnorm.go:434-442
    case GN_LAYER_SWIGLU:                                     // swiglu.go:295-308
      b.add("w", {d.out_size, d.in_size});
      b.add("v", {d.out_size, d.in_size});
      return;
    case GN_LAYER_TRANSFORMER: {  // transformer.go:786-801, 1402-1426
      const int64_t D = d.dim, FF = d.ff_dim;
      for (const char *w : {"wQ_", "wK_", "wV_", "wOut_"}) b.dense(std::string("mha_") + w, D, D);
      for (const char *nm : {"norm1_", "norm2_"}) {
        b.add(std::string(nm) + "gamma", {D});
        if (d.block_norm != GN_BLOCK_NORM_RMS) b.add(std::string(nm) + "beta", {D});
      }
      if (d.block_act == GN_BLOCK_ACT_SWIGLU) {
        b.add("ff1_w", {FF, D});
        b.add("ff1_v", {FF, D});
      } else {
        b.dense("ff1_", D, FF);
      }
      b.dense("ff2_", FF, D);
      return;
    }
    case GN_LAYER_BATCHNORM2D: {  // batchnorm2d.go:755-767: running stats first
      const int64_t C = d.in_channels;
      Tensor m;
      m.name = "running_mean"; m.shape = {C}; m.src = 1; m.layer = i; m.n = C;
      v.push_back(m);
      m.name = "running_var"; m.src = 2;
      v.push_back(m);
      if (pcount) {
        b.add("gamma", {C});
        b.add("beta", {C});
      }
      return;
    }
    default:  // no NamedParams: one flat tensor of Params() when there are any
      if (pcount > 0) b.add("params", {pcount});
      return;
  }
}

// Tensors of the whole model with the SaveBinaryWeights prefixes
int model_tensors(gn_model *M, std::vector<Tensor> &v) {
  for (int i = 0; i < model_layer_count(M); ++i) {
    int64_t off = 0, cnt = 0;
    int rc = gn_model_layer_params(M, i, &off, &cnt);
    if (rc) return rc;
    const size_t first = v.size();
    layer_tensors(M, i, off, cnt, v);
    int64_t arena = 0;
    for (size_t k = first; k < v.size(); ++k)
      if (v[k].src == 0) arena += v[k].n;
    if (arena != cnt)
      return model_error(M, GN_ERR_INVALID, "layer %d: named tensors cover %lld of %lld parameters", i,
                         (long long)arena, (long long)cnt);
  }
  return GN_OK;
}

int read_tensor(gn_model *M, const Tensor &t, std::vector<float> &data) {
  data.resize((size_t)t.n);
  if (t.src == 0) return gn_model_get_params(M, data.data(), t.off, t.n);
  std::vector<float> other((size_t)t.n);
  return t.src == 1 ? gn_model_get_running_stats(M, t.layer, data.data(), other.data(), (int32_t)t.n)
                    : gn_model_get_running_stats(M, t.layer, other.data(), data.data(), (int32_t)t.n);
}

struct File {
  FILE *f = nullptr;
  explicit File(const char *path, const char *mode) { f = path ? fopen(path, mode) : nullptr; }
  ~File() {
    if (f) fclose(f);
  }
  bool put(const void *p, size_t n) { return fwrite(p, 1, n, f) == n; }
  bool get(void *p, size_t n) { return fread(p, 1, n, f) == n; }
  template <class T> bool put_v(T v) { return put(&v, sizeof v); }  // little-endian host
  template <class T> bool get_v(T &v) { return get(&v, sizeof v); }
};

// Float32ToFloat16 (gguf.go): the mantissa is truncated, not rounded;
// exponents below the half range flush through the subnormal shift or to 0;
// NaN keeps a set low bit.
uint16_t f32_to_f16(float x) {
  uint32_t bits;
  memcpy(&bits, &x, 4);
  const uint16_t s = (uint16_t)((bits >> 16) & 0x8000);
  int e = (int)((bits >> 23) & 0xFF);
  uint32_t m = bits & 0x7FFFFF;
  if (e == 0) return s;
  if (e == 0xFF) return m == 0 ? (uint16_t)(s | 0x7C00) : (uint16_t)(s | 0x7C00 | (m >> 13) | 1);
  e -= 127 - 15;
  if (e >= 31) return (uint16_t)(s | 0x7C00);
  if (e <= 0) {
    if (e < -10) return s;
    m |= 0x800000;
    m >>= (uint32_t)(1 - e);
    return (uint16_t)(s | (m >> 13));
  }
  return (uint16_t)(s | (e << 10) | (m >> 13));
}

void replace_all(std::string &s, const char *from, const char *to) {
  const size_t fl = strlen(from), tl = strlen(to);
  for (size_t p = s.find(from); p != std::string::npos; p = s.find(from, p + tl)) s.replace(p, fl, to);
}

}  // namespace

extern "C" int gn_model_save_binary_weights(gn_model *M, const char *path) {
  if (!M) return GN_ERR_INVALID;
  std::vector<Tensor> ts;
  int rc = model_tensors(M, ts);
  if (rc) return rc;
  File f(path, "wb");
  if (!f.f) return model_error(M, GN_ERR_INVALID, "cannot create %s", path ? path : "(null)");
  bool ok = f.put("GONN", 4) && f.put_v<int32_t>(1) && f.put_v<int32_t>((int32_t)ts.size());
  std::vector<float> data;
  for (const Tensor &t : ts) {
    if ((rc = read_tensor(M, t, data))) return rc;
    char pre[64];
    snprintf(pre, sizeof pre, "layer_%d_%s_", t.layer, layer_type(model_layer_desc(M, t.layer)->kind));
    const std::string name = pre + t.name;
    ok = ok && f.put_v<int32_t>((int32_t)name.size()) && f.put(name.data(), name.size()) &&
         f.put_v<int32_t>((int32_t)t.shape.size());
    for (int64_t d : t.shape) ok = ok && f.put_v<int32_t>((int32_t)d);
    ok = ok && f.put_v<int32_t>((int32_t)t.n) && f.put(data.data(), data.size() * 4);
  }
  return ok ? GN_OK : model_error(M, GN_ERR_INVALID, "write to %s failed", path);
}

extern "C" int gn_model_load_binary_weights(gn_model *M, const char *path) {
  if (!M) return GN_ERR_INVALID;
  std::vector<Tensor> ts;
  int rc = model_tensors(M, ts);
  if (rc) return rc;
  File f(path, "rb");
  if (!f.f) return model_error(M, GN_ERR_INVALID, "cannot open %s", path ? path : "(null)");
  char magic[4];
  int32_t ver = 0, count = 0;
  if (!f.get(magic, 4) || memcmp(magic, "GONN", 4) || !f.get_v(ver) || ver != 1 || !f.get_v(count))
    return model_error(M, GN_ERR_INVALID, "%s: not a GONN version 1 weights file", path);
  if (count != (int32_t)ts.size())
    return model_error(M, GN_ERR_SHAPE, "%s holds %d tensors, this model %d", path, count, (int)ts.size());
  // read everything first so that a bad file leaves the model untouched
  std::vector<std::vector<float>> all(ts.size());
  for (size_t k = 0; k < ts.size(); ++k) {
    const Tensor &t = ts[k];
    char pre[64];
    snprintf(pre, sizeof pre, "layer_%d_%s_", t.layer, layer_type(model_layer_desc(M, t.layer)->kind));
    const std::string want = pre + t.name;
    int32_t nl = 0, rank = 0, len = 0;
    if (!f.get_v(nl) || nl < 0 || nl > 4096) return model_error(M, GN_ERR_INVALID, "%s: bad name", path);
    std::string name((size_t)nl, '\0');
    if (!f.get(&name[0], (size_t)nl) || !f.get_v(rank) || rank < 0 || rank > 16)
      return model_error(M, GN_ERR_INVALID, "%s: truncated tensor header", path);
    for (int r = 0; r < rank; ++r) {
      int32_t dim;
      if (!f.get_v(dim)) return model_error(M, GN_ERR_INVALID, "%s: truncated shape", path);
    }
    if (!f.get_v(len)) return model_error(M, GN_ERR_INVALID, "%s: truncated length", path);
    if (name != want || len != t.n)
      return model_error(M, GN_ERR_SHAPE, "%s: tensor %zu is %s[%d], expected %s[%lld]", path, k,
                         name.c_str(), len, want.c_str(), (long long)t.n);
    all[k].resize((size_t)len);
    if (!f.get(all[k].data(), (size_t)len * 4))
      return model_error(M, GN_ERR_INVALID, "%s: truncated data of %s", path, name.c_str());
  }
  for (size_t k = 0; k < ts.size(); ++k) {
    const Tensor &t = ts[k];
    if (t.src == 0) {
      if ((rc = gn_model_set_params(M, all[k].data(), t.off, t.n))) return rc;
    } else if (t.src == 1) {  // running_mean then running_var, adjacent
      if ((rc = gn_model_set_running_stats(M, t.layer, all[k].data(), all[k + 1].data(), (int32_t)t.n)))
        return rc;
    }
  }
  return GN_OK;
}

extern "C" int gn_model_save_gguf(gn_model *M, const char *path, int32_t f16) {
  if (!M) return GN_ERR_INVALID;
  if (f16 != 0 && f16 != 1) return model_error(M, GN_ERR_INVALID, "GGUF tensor type %d", f16);
  std::vector<Tensor> ts;
  int rc = model_tensors(M, ts);
  if (rc) return rc;
  std::vector<std::string> names;
  for (const Tensor &t : ts) {
    std::string n = t.name;
    if (n == "params") {
      n = "weight";  // the flat fallback (net.go:1277-1285)
    } else {                               // net.go:1254-1269, applied in this order
      replace_all(n, "weights", "weight");
      replace_all(n, "biases", "bias");
      replace_all(n, "gamma", "weight");
      replace_all(n, "beta", "bias");
      replace_all(n, "mha_wQ_", "attn_q.");
      replace_all(n, "mha_wK_", "attn_k.");
      replace_all(n, "mha_wV_", "attn_v.");
      replace_all(n, "mha_wOut_", "attn_output.");
      replace_all(n, "ff1_", "ffn_up.");
      replace_all(n, "ff2_", "ffn_down.");
      replace_all(n, "norm1_", "attn_norm.");
      replace_all(n, "norm2_", "ffn_norm.");
    }
    names.push_back("blk." + std::to_string(t.layer) + "." + n);
  }
  const std::string loss = model_loss_kind(M) == GN_LOSS_MSE ? "loss.MSE" : "loss.CrossEntropy";
  const std::string arch = "goneuron", gname = "GoNeuron Model";
  const uint64_t align = 32;
  File f(path, "wb");
  if (!f.f) return model_error(M, GN_ERR_INVALID, "cannot create %s", path ? path : "(null)");
  auto str = [&](const std::string &s) { return f.put_v<uint64_t>(s.size()) && f.put(s.data(), s.size()); };
  auto kv_str = [&](const char *k, const std::string &v) {
    return str(k) && f.put_v<uint32_t>(8) && str(v);
  };
  auto kv_u32 = [&](const char *k, uint32_t v) { return str(k) && f.put_v<uint32_t>(4) && f.put_v<uint32_t>(v); };
  bool ok = f.put_v<uint32_t>(0x46554747u) && f.put_v<uint32_t>(3) && f.put_v<uint64_t>(ts.size()) &&
            f.put_v<uint64_t>(5);
  ok = ok && kv_str("general.architecture", arch) && kv_str("general.name", gname) &&
       kv_u32("general.alignment", 32) && kv_u32("goneuron.layer_count", (uint32_t)model_layer_count(M)) &&
       kv_str("goneuron.loss_type", loss);
  const uint64_t esz = f16 ? 2 : 4;
  uint64_t cur = 0;
  for (size_t k = 0; k < ts.size(); ++k) {  // dims last-first, offsets aligned (gguf.go:174-195)
    ok = ok && str(names[k]) && f.put_v<uint32_t>((uint32_t)ts[k].shape.size());
    for (size_t r = ts[k].shape.size(); r-- > 0;) ok = ok && f.put_v<uint64_t>((uint64_t)ts[k].shape[r]);
    ok = ok && f.put_v<uint32_t>((uint32_t)f16) && f.put_v<uint64_t>(cur);
    cur += (uint64_t)ts[k].n * esz;
    cur = (cur + align - 1) & ~(align - 1);
  }
  std::vector<float> data;
  std::vector<uint16_t> half;
  static const char zeros[32] = {0};
  long pos = ftell(f.f);
  ok = ok && pos >= 0 && f.put(zeros, (size_t)((align - (uint64_t)pos % align) % align));
  for (const Tensor &t : ts) {
    if ((rc = read_tensor(M, t, data))) return rc;
    pos = ftell(f.f);
    ok = ok && pos >= 0 && f.put(zeros, (size_t)((align - (uint64_t)pos % align) % align));
    if (f16) {
      half.resize(data.size());
      for (size_t j = 0; j < data.size(); ++j) half[j] = f32_to_f16(data[j]);
      ok = ok && f.put(half.data(), half.size() * 2);
    } else {
      ok = ok && f.put(data.data(), data.size() * 4);
    }
  }
  return ok ? GN_OK : model_error(M, GN_ERR_INVALID, "write to %s failed", path);
}

// State file: "GNST", u32 version 1, i64 nparams, i32 layers, i32 timestep,
// params, Adam m, Adam v (nparams floats each), then per layer i32 kind and,
// for BatchNorm2D, i32 C + mean + var, for MoE, u32 count + the stream states.
extern "C" int gn_model_save_state(gn_model *M, const char *path) {
  if (!M) return GN_ERR_INVALID;
  int64_t n = 0;
  int rc = gn_model_nparams(M, &n);
  if (rc) return rc;
  std::vector<float> p((size_t)std::max<int64_t>(n, 1)), m(p.size()), v(p.size());
  int32_t t = 0;
  if ((rc = gn_model_get_params(M, p.data(), 0, n)) || (rc = gn_model_get_adam(M, m.data(), v.data(), 0, n, &t)))
    return rc;
  File f(path, "wb");
  if (!f.f) return model_error(M, GN_ERR_INVALID, "cannot create %s", path ? path : "(null)");
  const int L = model_layer_count(M);
  bool ok = f.put("GNST", 4) && f.put_v<uint32_t>(1) && f.put_v<int64_t>(n) && f.put_v<int32_t>(L) &&
            f.put_v<int32_t>(t) && f.put(p.data(), (size_t)n * 4) && f.put(m.data(), (size_t)n * 4) &&
            f.put(v.data(), (size_t)n * 4);
  for (int i = 0; i < L && ok; ++i) {
    const gn_layer_desc &d = *model_layer_desc(M, i);
    ok = f.put_v<int32_t>(d.kind);
    if (d.kind == GN_LAYER_BATCHNORM2D) {
      std::vector<float> a((size_t)d.in_channels), b(a.size());
      if ((rc = gn_model_get_running_stats(M, i, a.data(), b.data(), d.in_channels))) return rc;
      ok = ok && f.put_v<int32_t>(d.in_channels) && f.put(a.data(), a.size() * 4) && f.put(b.data(), b.size() * 4);
    }
    if (std::vector<uint64_t> *s = model_noise_streams(M, i))
      ok = ok && f.put_v<uint32_t>((uint32_t)s->size()) && f.put(s->data(), s->size() * 8);
  }
  return ok ? GN_OK : model_error(M, GN_ERR_INVALID, "write to %s failed", path);
}

extern "C" int gn_model_load_state(gn_model *M, const char *path) {
  if (!M) return GN_ERR_INVALID;
  int64_t n = 0;
  int rc = gn_model_nparams(M, &n);
  if (rc) return rc;
  File f(path, "rb");
  if (!f.f) return model_error(M, GN_ERR_INVALID, "cannot open %s", path ? path : "(null)");
  char magic[4];
  uint32_t ver = 0;
  int64_t fn = 0;
  int32_t L = 0, t = 0;
  if (!f.get(magic, 4) || memcmp(magic, "GNST", 4) || !f.get_v(ver) || ver != 1 || !f.get_v(fn) ||
      !f.get_v(L) || !f.get_v(t))
    return model_error(M, GN_ERR_INVALID, "%s: not a version 1 state file", path);
  if (fn != n || L != model_layer_count(M) || t < 0)
    return model_error(M, GN_ERR_SHAPE, "%s: %lld parameters / %d layers, this model %lld / %d", path,
                       (long long)fn, L, (long long)n, model_layer_count(M));
  std::vector<float> p((size_t)std::max<int64_t>(n, 1)), m(p.size()), v(p.size());
  if (!f.get(p.data(), (size_t)n * 4) || !f.get(m.data(), (size_t)n * 4) || !f.get(v.data(), (size_t)n * 4))
    return model_error(M, GN_ERR_INVALID, "%s: truncated", path);
  struct Extra { int layer; std::vector<float> mean, var; std::vector<uint64_t> rng; };
  std::vector<Extra> extra;
  for (int i = 0; i < L; ++i) {
    const gn_layer_desc &d = *model_layer_desc(M, i);
    int32_t kind = 0;
    if (!f.get_v(kind) || kind != d.kind)
      return model_error(M, GN_ERR_SHAPE, "%s: layer %d kind %d, this model %d", path, i, kind, d.kind);
    Extra e{i, {}, {}, {}};
    if (d.kind == GN_LAYER_BATCHNORM2D) {
      int32_t C = 0;
      if (!f.get_v(C) || C != d.in_channels) return model_error(M, GN_ERR_SHAPE, "%s: channels", path);
      e.mean.resize((size_t)C);
      e.var.resize((size_t)C);
      if (!f.get(e.mean.data(), (size_t)C * 4) || !f.get(e.var.data(), (size_t)C * 4))
        return model_error(M, GN_ERR_INVALID, "%s: truncated", path);
    }
    if (std::vector<uint64_t> *s = model_noise_streams(M, i)) {
      uint32_t cnt = 0;
      if (!f.get_v(cnt) || cnt != s->size()) return model_error(M, GN_ERR_SHAPE, "%s: noise streams", path);
      e.rng.resize(cnt);
      if (!f.get(e.rng.data(), (size_t)cnt * 8)) return model_error(M, GN_ERR_INVALID, "%s: truncated", path);
    }
    extra.push_back(std::move(e));
  }
  if ((rc = gn_model_set_params(M, p.data(), 0, n)) || (rc = gn_model_set_adam(M, m.data(), v.data(), 0, n, t)))
    return rc;
  for (Extra &e : extra) {
    if (!e.mean.empty() &&
        (rc = gn_model_set_running_stats(M, e.layer, e.mean.data(), e.var.data(), (int32_t)e.mean.size())))
      return rc;
    if (!e.rng.empty()) *model_noise_streams(M, e.layer) = e.rng;
  }
  return GN_OK;
}
