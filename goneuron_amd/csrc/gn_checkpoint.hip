// Checkpoint formats around the device-resident arena (host code).
//
//  - SaveBinaryWeights (net.go:1119-1214) and a reader for it;
//  - SaveGGUF / SaveGGUFExt (net.go:1217-1392, gguf.go): GGUF v3, F32 or F16;
//  - a full training-state file for resume (parameters, Adam moments and
//    timestep, BatchNorm2D running statistics, MoE noise streams);
//  - Network.Save / net.Load (net.go:863-1075): the "GONN" gob file.
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
#include <climits>
#include <cmath>
#include <map>
#include <string>
#include <vector>

#include "gn_common.h"
#include "gn_ctx.h"

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
    case GN_LAYER_LAYERNORM: return "LayerNorm";
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
    case GN_LAYER_LAYERNORM:                                  // layernorm.go:533-550
      b.add("gamma", {d.dim});
      b.add("beta", {d.dim});
      return;
    case GN_LAYER_MHA: {  // transformer.go:786-801; pcount = 4 (D^2 + D)
      const int64_t D = (int64_t)((sqrt(1.0 + (double)pcount) - 1.0) / 2.0 + 0.5);
      for (const char *w : {"wQ_", "wK_", "wV_", "wOut_"}) b.dense(w, D, D);
      return;
    }
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

// ---------------------------------------------------------------------------
// Network.Save / net.Load (net.go:863-1075): "GONN", int32 1 (little endian),
// then an encoding/gob stream of the layer count (int32), the loss name, the
// optimizer name, one LayerConfig per layer (net.go:1393-1423, filled by
// ExtractLayerConfig net.go:1425-1505), the flat parameters ([]float32) and
// Adam's GobState (opt.go:262-322).
//
// gob wire format (encoding/gob package documentation): a stream of
// messages, each an unsigned byte count then a signed type id; a negative id
// carries the definition (a wireType value) of type -id, a positive one a
// value of that type.  Unsigned integers below 128 take one byte, larger ones
// a byte holding minus the byte count and then the big-endian bytes without
// leading zeros; signed integers are folded (bit 0 = sign, the rest
// complemented when negative); floats are the float64 bits byte-reversed and
// sent as unsigned; strings and byte slices are a count then the bytes.
// Struct fields are (field-number delta, value) pairs, zero-valued fields
// left out, ending with delta 0; a top-level value that is not a struct is
// preceded by a zero delta.  Type ids below 64 are gob's own (bool 1, int 2,
// uint 3, float 4, []byte 5, string 6, complex 7, interface 8); user types are
// numbered from 64 in the order a process first meets them, a struct before
// its fields' types.
// ---------------------------------------------------------------------------
namespace {
namespace gob {

enum : int64_t { T_BOOL = 1, T_INT = 2, T_UINT = 3, T_FLOAT = 4, T_BYTES = 5, T_STRING = 6,
                 T_COMPLEX = 7, T_INTERFACE = 8 };

struct Out {
  std::string b;
  void u(uint64_t x) {
    if (x < 128) {
      b.push_back((char)x);
      return;
    }
    unsigned char t[8];
    int n = 0;
    for (; x; x >>= 8) t[n++] = (unsigned char)(x & 0xFF);
    b.push_back((char)(unsigned char)(256 - n));
    while (n) b.push_back((char)t[--n]);
  }
  void i(int64_t v) { u(v < 0 ? ((uint64_t)~v << 1) | 1 : (uint64_t)v << 1); }
  void f(double d) {
    uint64_t x;
    memcpy(&x, &d, 8);
    u(__builtin_bswap64(x));
  }
  void s(const std::string &v) {
    u(v.size());
    b += v;
  }
  void message(const Out &m) {  // byte count, then the message
    u(m.b.size());
    b += m.b;
  }
};

// struct value writer: field-number deltas, zero values left out
struct Fields {
  Out &o;
  int last = -1;
  void at(int k) {
    o.u((uint64_t)(k - last));
    last = k;
  }
  void i(int k, int64_t v) {
    if (v) at(k), o.i(v);
  }
  void f(int k, float v) {
    if (v != 0.f) at(k), o.f((double)v);
  }
  void s(int k, const std::string &v) {
    if (!v.empty()) at(k), o.s(v);
  }
  void b(int k, bool v) {
    if (v) at(k), o.u(1);
  }
  void end() { o.u(0); }
};

// CommonType{Name, Id} (an anonymous slice type has no name)
void common(Out &m, const std::string &name, int64_t id) {
  Fields f{m};
  f.s(0, name);
  f.i(1, id);
  f.end();
}

// wireType{StructT: &structType{CommonType{name, id}, Field: fields}}
Out struct_def(int64_t id, const std::string &name, const std::vector<std::pair<std::string, int64_t>> &fields) {
  Out m;
  m.i(-id);
  Fields w{m};
  w.at(2);  // StructT
  Fields st{m};
  st.at(0);
  common(m, name, id);
  st.at(1);
  m.u(fields.size());
  for (const auto &f : fields) {
    Fields ft{m};
    ft.s(0, f.first);
    ft.i(1, f.second);
    ft.end();
  }
  st.end();
  w.end();
  return m;
}

// wireType{SliceT: &sliceType{CommonType{name, id}, Elem: elem}}
Out slice_def(int64_t id, const std::string &name, int64_t elem) {
  Out m;
  m.i(-id);
  Fields w{m};
  w.at(1);  // SliceT
  Fields st{m};
  st.at(0);
  common(m, name, id);
  st.i(1, elem);
  st.end();
  w.end();
  return m;
}

void floats(Out &m, const float *p, size_t n) {
  m.u(n);
  for (size_t k = 0; k < n; ++k) m.f((double)p[k]);
}

// ---- reading ----
struct In {
  const uint8_t *p = nullptr, *e = nullptr;
  bool ok = true;
  uint64_t fail() {
    ok = false;
    p = e;
    return 0;
  }
  size_t left() const { return (size_t)(e - p); }
  uint64_t u() {
    if (p >= e) return fail();
    const uint8_t b = *p++;
    if (b < 128) return b;
    const int n = 256 - b;
    if (n > 8 || (int)left() < n) return fail();
    uint64_t x = 0;
    for (int k = 0; k < n; ++k) x = x << 8 | *p++;
    return x;
  }
  int64_t i() {
    const uint64_t x = u();
    return (x & 1) ? ~(int64_t)(x >> 1) : (int64_t)(x >> 1);
  }
  double f() {
    const uint64_t x = __builtin_bswap64(u());
    double d;
    memcpy(&d, &x, 8);
    return d;
  }
  bool str(std::string &s) {
    const uint64_t n = u();
    if (!ok || n > left()) return fail(), false;
    s.assign((const char *)p, (size_t)n);
    p += n;
    return true;
  }
  bool skip_bytes() {
    const uint64_t n = u();
    if (!ok || n > left()) return fail(), false;
    p += n;
    return true;
  }
};

struct WireType {
  int kind = 0;  // 1 array, 2 slice, 3 struct, 4 map, 5 GobEncoder / BinaryMarshaler / TextMarshaler
  std::string name;
  int64_t elem = 0, key = 0, len = 0;
  std::vector<std::pair<std::string, int64_t>> fields;
};

struct Decoder {
  In s;  // the stream after "GONN" and the version
  std::map<int64_t, WireType> types;
  std::string err;

  bool bad(const char *what) {
    if (err.empty()) err = what;
    return false;
  }

  // CommonType and the types built on it; unknown fields make the definition bad
  bool common(In &m, std::string &name, int64_t &id) {
    for (int f = -1;;) {
      const uint64_t d = m.u();
      if (!m.ok) return false;
      if (d == 0) return true;
      f += (int)d;
      if (f == 0) m.str(name);
      else if (f == 1) id = m.i();
      else return false;
    }
  }
  bool definition(In &m, WireType &w, int64_t &id) {
    int f = -1;
    for (;;) {
      const uint64_t d = m.u();
      if (!m.ok) return false;
      if (d == 0) break;
      f += (int)d;
      if (f < 0 || f > 6 || w.kind) return false;
      w.kind = f == 0 ? 1 : f == 1 ? 2 : f == 2 ? 3 : f == 3 ? 4 : 5;
      for (int g = -1;;) {  // the arrayType / sliceType / structType / mapType / gobEncoderType
        const uint64_t e = m.u();
        if (!m.ok) return false;
        if (e == 0) break;
        g += (int)e;
        if (g == 0) {
          if (!common(m, w.name, id)) return false;
        } else if (w.kind == 1 && g == 1) w.elem = m.i();
        else if (w.kind == 1 && g == 2) w.len = m.i();
        else if (w.kind == 2 && g == 1) w.elem = m.i();
        else if (w.kind == 4 && g == 1) w.key = m.i();
        else if (w.kind == 4 && g == 2) w.elem = m.i();
        else if (w.kind == 3 && g == 1) {
          const uint64_t n = m.u();
          if (!m.ok || n > m.left()) return false;
          for (uint64_t k = 0; k < n; ++k) {
            std::pair<std::string, int64_t> fl;
            for (int h = -1;;) {
              const uint64_t q = m.u();
              if (!m.ok) return false;
              if (q == 0) break;
              h += (int)q;
              if (h == 0) m.str(fl.first);
              else if (h == 1) fl.second = m.i();
              else return false;
            }
            w.fields.push_back(fl);
          }
        } else return false;
      }
    }
    return m.ok && w.kind != 0 && id > 0;
  }

  // The next value message: definitions before it are recorded; returns its
  // type id and leaves `m` at the value
  bool next(In &m, int64_t &id) {
    for (;;) {
      const uint64_t n = s.u();
      if (!s.ok) return bad("unexpected end of the gob stream");
      if (n == 0 || n > s.left()) return bad("gob message length out of range");
      m = In{s.p, s.p + n};
      s.p += n;
      const int64_t t = m.i();
      if (!m.ok || t == 0) return bad("bad gob type id");
      if (t > 0) {
        id = t;
        return true;
      }
      WireType w;
      int64_t wid = 0;
      if (!definition(m, w, wid) || wid != -t) return bad("bad gob type definition");
      types[wid] = std::move(w);
    }
  }

  const WireType *wire(int64_t id) {
    auto it = types.find(id);
    return it == types.end() ? nullptr : &it->second;
  }

  // reads past one value of type `id`
  bool skip(In &m, int64_t id, int depth = 0) {
    if (depth > 32) return false;
    switch (id) {
      case T_BOOL: case T_INT: case T_UINT: case T_FLOAT: m.u(); return m.ok;
      case T_COMPLEX: m.u(); m.u(); return m.ok;
      case T_BYTES: case T_STRING: return m.skip_bytes();
      default: break;
    }
    const WireType *w = wire(id);
    if (!w) return false;
    switch (w->kind) {
      case 1: case 2: {
        const uint64_t n = m.u();
        if (!m.ok || (w->kind == 1 && (int64_t)n != w->len) || n > m.left()) return false;
        for (uint64_t k = 0; k < n; ++k)
          if (!skip(m, w->elem, depth + 1)) return false;
        return true;
      }
      case 3:
        for (int f = -1;;) {
          const uint64_t d = m.u();
          if (!m.ok) return false;
          if (d == 0) return true;
          f += (int)d;
          if (f < 0 || f >= (int)w->fields.size() || !skip(m, w->fields[f].second, depth + 1)) return false;
        }
      case 4: {
        const uint64_t n = m.u();
        if (!m.ok || n > m.left()) return false;
        for (uint64_t k = 0; k < n; ++k)
          if (!skip(m, w->key, depth + 1) || !skip(m, w->elem, depth + 1)) return false;
        return true;
      }
      default: return m.skip_bytes();
    }
  }

  // singleton values: a zero field delta, then the value
  bool singleton(In &m) {
    if (m.u() != 0 || !m.ok) return bad("gob: corrupted data: non-zero delta for singleton");
    return true;
  }
  bool read_int(int64_t &v) {
    In m;
    int64_t id;
    if (!next(m, id)) return false;
    if (id != T_INT) return bad("gob: type mismatch (an int was expected)");
    if (!singleton(m)) return false;
    v = m.i();
    return m.ok || bad("gob: truncated int");
  }
  bool read_string(std::string &v) {
    In m;
    int64_t id;
    if (!next(m, id)) return false;
    if (id != T_STRING) return bad("gob: type mismatch (a string was expected)");
    return (singleton(m) && m.str(v)) || bad("gob: truncated string");
  }
  // a []float32 value: a slice whose elements are floats, each within float32 range
  bool float_slice(In &m, int64_t id, std::vector<float> &v) {
    const WireType *w = wire(id);
    if (!w || w->kind != 2 || w->elem != T_FLOAT) return bad("gob: type mismatch ([]float32 expected)");
    const uint64_t n = m.u();
    if (!m.ok || n > m.left()) return bad("gob: truncated []float32");
    v.resize((size_t)n);
    for (uint64_t k = 0; k < n; ++k) {
      const double d = m.f();
      if (std::fabs(d) > 3.4028234663852886e38 && std::isfinite(d)) return bad("gob: float32 value out of range");
      v[(size_t)k] = (float)d;
    }
    return m.ok || bad("gob: truncated []float32");
  }
  bool read_floats(std::vector<float> &v) {
    In m;
    int64_t id;
    return next(m, id) && singleton(m) && float_slice(m, id, v);
  }
};

// LayerConfig (net.go:1393-1423)
struct LayerConfig {
  std::string type, activation;
  int64_t in_size = 0, out_size = 0, kernel = 0, stride = 0, padding = 0, in_channels = 0,
          out_channels = 0, normalized_shape = 0, num_centers = 0;
  float alpha = 0, prob = 0, eps = 0, gamma = 0;
  bool affine = false;
  std::vector<float> params;
};

bool read_config(Decoder &D, LayerConfig &c) {
  In m;
  int64_t id;
  if (!D.next(m, id)) return false;
  const WireType *w = D.wire(id);
  if (!w || w->kind != 3) return D.bad("gob: type mismatch (LayerConfig expected)");
  for (int f = -1;;) {
    const uint64_t d = m.u();
    if (!m.ok) return D.bad("gob: truncated LayerConfig");
    if (d == 0) return true;
    f += (int)d;
    if (f < 0 || f >= (int)w->fields.size()) return D.bad("gob: LayerConfig field out of range");
    const std::string &name = w->fields[f].first;
    const int64_t t = w->fields[f].second;
    auto want = [&](int64_t ty) { return t == ty || D.bad("gob: wrong type for a LayerConfig field"); };
    int64_t *iv = name == "InSize" ? &c.in_size : name == "OutSize" ? &c.out_size
                : name == "KernelSize" ? &c.kernel : name == "Stride" ? &c.stride
                : name == "Padding" ? &c.padding : name == "InChannels" ? &c.in_channels
                : name == "OutChannels" ? &c.out_channels : name == "NormalizedShape" ? &c.normalized_shape
                : name == "NumCenters" ? &c.num_centers : nullptr;
    float *fv = name == "Alpha" ? &c.alpha : name == "Prob" ? &c.prob : name == "Eps" ? &c.eps
              : name == "Gamma" ? &c.gamma : nullptr;
    if (iv) {
      if (!want(T_INT)) return false;
      *iv = m.i();
    } else if (fv) {
      if (!want(T_FLOAT)) return false;
      const double x = m.f();
      if (std::fabs(x) > 3.4028234663852886e38 && std::isfinite(x)) return D.bad("gob: float32 value out of range");
      *fv = (float)x;
    } else if (name == "Type" || name == "Activation") {
      if (!want(T_STRING) || !m.str(name == "Type" ? c.type : c.activation)) return D.bad("gob: truncated string");
    } else if (name == "Affine") {
      if (!want(T_BOOL)) return false;
      c.affine = m.u() != 0;
    } else if (name == "Params") {
      if (!D.float_slice(m, t, c.params)) return false;
    } else if (!D.skip(m, t)) {
      return D.bad("gob: bad LayerConfig field");
    }
    if (!m.ok) return D.bad("gob: truncated LayerConfig");
  }
}

}  // namespace gob

// getActivationType (net.go:1622-1651) for the activations built here; a
// nil activation takes the default case
const char *activation_name(int act) {
  switch (act) {
    case GN_ACT_SIGMOID: return "Sigmoid";
    case GN_ACT_TANH: return "Tanh";
    case GN_ACT_SOFTMAX: return "Softmax";
    case GN_ACT_LOGSOFTMAX: return "LogSoftmax";
    case GN_ACT_LINEAR: return "Linear";
    case GN_ACT_GELU: return "GELU";
    default: return "ReLU";
  }
}

// createActivation (net.go:1590-1619): value activations; names this
// library does not build give -1, unknown names the default ReLU
int activation_code(const std::string &s) {
  if (s == "Sigmoid") return GN_ACT_SIGMOID;
  if (s == "Tanh") return GN_ACT_TANH;
  if (s == "Softmax") return GN_ACT_SOFTMAX;
  if (s == "LogSoftmax") return GN_ACT_LOGSOFTMAX;
  if (s == "Linear") return GN_ACT_LINEAR;
  if (s == "GELU") return GN_ACT_GELU;
  if (s == "LeakyReLU" || s == "PReLU" || s == "ELU" || s == "SiLU" || s == "SELU") return -1;
  return GN_ACT_RELU;
}

}  // namespace

// Network.Encode (net.go:1008-1075).  Type ids are those a Go process gives
// when this is its first use of gob: LayerConfig 64, []float32 65,
// adamGobState 66, [][]float32 67.
extern "C" int gn_model_save_gob(gn_model *M, const char *path) {
  using namespace gob;
  if (!M) return GN_ERR_INVALID;
  int64_t n = 0;
  int rc = gn_model_nparams(M, &n);
  if (rc) return rc;
  std::vector<float> p((size_t)std::max<int64_t>(n, 1)), am(p.size()), av(p.size());
  int32_t t = 0;
  if ((rc = gn_model_get_params(M, p.data(), 0, n)) || (rc = gn_model_get_adam(M, am.data(), av.data(), 0, n, &t)))
    return rc;
  const int L = model_layer_count(M);
  const int64_t ID_CFG = 64, ID_F32S = 65, ID_ADAM = 66, ID_F32SS = 67;
  Out s;
  {
    Out m;
    m.i(T_INT), m.u(0), m.i(L);
    s.message(m);
  }
  {
    Out m;  // net.go:1024-1036: MSE or CrossEntropy here
    m.i(T_STRING), m.u(0), m.s(model_loss_kind(M) == GN_LOSS_CE ? "CrossEntropy" : "MSE");
    s.message(m);
  }
  {
    Out m;
    m.i(T_STRING), m.u(0), m.s("Adam");
    s.message(m);
  }
  s.message(struct_def(ID_CFG, "LayerConfig",
                       {{"Type", T_STRING}, {"InSize", T_INT}, {"OutSize", T_INT}, {"Params", ID_F32S},
                        {"Activation", T_STRING}, {"Alpha", T_FLOAT}, {"KernelSize", T_INT}, {"Stride", T_INT},
                        {"Padding", T_INT}, {"InChannels", T_INT}, {"OutChannels", T_INT}, {"Prob", T_FLOAT},
                        {"Eps", T_FLOAT}, {"Affine", T_BOOL}, {"NormalizedShape", T_INT},
                        {"NumCenters", T_INT}, {"Gamma", T_FLOAT}}));
  s.message(slice_def(ID_F32S, "[]float32", T_FLOAT));
  const bool dims = model_master_dims(M);
  for (int i = 0; i < L; ++i) {
    const gn_layer_desc &d = *model_layer_desc(M, i);
    int64_t off = 0, cnt = 0;
    if ((rc = gn_model_layer_params(M, i, &off, &cnt))) return rc;
    ConvShape cs{};
    PoolShape ps{};
    float eps = 0;
    model_layer_geom(M, i, &cs, &ps, &eps);
    // ExtractLayerConfig (net.go:1426-1505)
    int64_t in = -1, out = -1, k = 0, st = 0, pad = 0, inC = 0, outC = 0, ns = 0;
    float prob = 0, e = 0;
    bool affine = false;
    std::string act;
    switch (d.kind) {
      case GN_LAYER_DENSE:
        in = d.in_size, out = d.out_size, act = activation_name(d.act);
        break;
      case GN_LAYER_CONV2D:  // OutSize() is outC x oH x oW once the input size is known (conv2d.go:1346-1353)
        inC = cs.inC, outC = dims ? (int64_t)cs.outC * cs.oH * cs.oW : cs.outC;
        k = cs.k, st = cs.stride, pad = cs.pad, act = activation_name(d.act);
        break;
      case GN_LAYER_DROPOUT:
        prob = d.p, in = d.in_size;
        break;
      case GN_LAYER_BATCHNORM2D:
        inC = d.in_channels, e = eps, affine = !d.no_affine;
        break;
      case GN_LAYER_MAXPOOL2D:  // InSize() / (k k), InSize() = C H W or 0 (maxpool2d.go:482-487)
        inC = (dims ? (int64_t)ps.C * ps.H * ps.W : 0) / ((int64_t)ps.k * ps.k);
        k = ps.k, st = ps.stride, pad = ps.pad;
        break;
      case GN_LAYER_AVGPOOL2D:  // a forward pass sets a lazy channel count to 1 (avgpool2d.go:100-103)
        inC = (dims && d.in_channels <= 0) ? 1 : d.in_channels;
        k = ps.k, st = ps.stride, pad = ps.pad;
        break;
      case GN_LAYER_EMBEDDING:
        in = d.vocab, out = d.dim;
        break;
      case GN_LAYER_LAYERNORM:  // net.go:1469-1473
        ns = d.dim, e = eps, affine = true;
        break;
      default:
        break;
    }
    Out m;
    m.i(ID_CFG);
    Fields f{m};
    f.s(0, layer_type(d.kind));
    f.i(1, in);
    f.i(2, out);
    if (cnt > 0) f.at(3), floats(m, p.data() + off, (size_t)cnt);
    f.s(4, act);
    f.i(6, k);
    f.i(7, st);
    f.i(8, pad);
    f.i(9, inC);
    f.i(10, outC);
    f.f(11, prob);
    f.f(12, e);
    f.b(13, affine);
    f.i(14, ns);
    f.end();
    s.message(m);
  }
  {
    Out m;
    m.i(ID_F32S), m.u(0), floats(m, p.data(), (size_t)n);
    s.message(m);
  }
  // Adam.GobState (opt.go:312-322): Network.Step hands StepInPlace the whole
  // flat buffer (net.go:260-284); above 1000 parameters its moments live in
  // mGlobal / vGlobal, which GobState leaves out, else in momentum1[0] /
  // momentum2[0] (opt.go:129-153).  A network without parameters steps each
  // layer on its own, leaving one empty moment slice per layer.
  s.message(struct_def(ID_ADAM, "adamGobState",
                       {{"LearningRate", T_FLOAT}, {"Beta1", T_FLOAT}, {"Beta2", T_FLOAT}, {"Epsilon", T_FLOAT},
                        {"Momentum1", ID_F32SS}, {"Momentum2", ID_F32SS}, {"Timestep", T_INT}}));
  s.message(slice_def(ID_F32SS, "[][]float32", ID_F32S));
  {
    const gn_adam_desc &a = model_adam(M);
    Out m;
    m.i(ID_ADAM);
    Fields f{m};
    f.f(0, a.lr);
    f.f(1, a.beta1);
    f.f(2, a.beta2);
    f.f(3, a.eps);
    if (t > 0 && n <= 1000) {
      for (int k = 4; k <= 5; ++k) {
        f.at(k);
        if (n > 0) {
          m.u(1);
          floats(m, (k == 4 ? am : av).data(), (size_t)n);
        } else {
          m.u((uint64_t)L);
          for (int l = 0; l < L; ++l) m.u(0);
        }
      }
    }
    f.i(6, t);
    f.end();
    s.message(m);
  }
  File file(path, "wb");
  if (!file.f) return model_error(M, GN_ERR_INVALID, "cannot create %s", path ? path : "(null)");
  const bool ok = file.put("GONN", 4) && file.put_v<int32_t>(1) && file.put(s.b.data(), s.b.size());
  return ok ? GN_OK : model_error(M, GN_ERR_INVALID, "write to %s failed", path);
}

// net.Load (net.go:875-1005) onto this device: the same checks in the same
// order, then CreateLayer (net.go:1512-1588) for each LayerConfig and a fresh
// Adam(0.001): the reference decodes the optimizer state into an `any`, which
// gob refuses for a struct, so the saved moments and timestep are never
// restored.  Layer types this library does not build (LayerNorm, RBF and bare
// LSTM / GRU, which the reference can rebuild; "Unknown", which it cannot), a
// Huber loss and an SGD optimizer are GN_ERR_UNSUPPORTED.  So is a layer whose
// saved parameter count differs from the layer its config describes (a
// Conv2D saved after a forward pass records outC x oH x oW output channels;
// the reference then builds that wider layer and copies the saved values
// into the front of its parameters).
extern "C" int gn_model_load_gob(gn_ctx *c, const char *path, int32_t in_len, int32_t max_batch,
                                 int32_t workers, gn_model **out, int32_t *loss_kind) {
  using namespace gob;
  if (!c || !out) return GN_ERR_INVALID;
  ENTRY(c);
  *out = nullptr;
  std::string buf;
  {
    File f(path, "rb");
    if (!f.f) return set_err(c, GN_ERR_INVALID, "failed to open file: %s", path ? path : "(null)");
    char tmp[1 << 16];
    for (size_t got; (got = fread(tmp, 1, sizeof tmp, f.f)) > 0;) buf.append(tmp, got);
  }
  if (buf.size() < 4) return set_err(c, GN_ERR_INVALID, "failed to read magic number");
  if (memcmp(buf.data(), "GONN", 4))
    return set_err(c, GN_ERR_INVALID, "invalid magic number: expected GONN, got %.4s", buf.data());
  int32_t version = 0;
  if (buf.size() < 8) return set_err(c, GN_ERR_INVALID, "failed to read version");
  memcpy(&version, buf.data() + 4, 4);
  if (version != 1) return set_err(c, GN_ERR_INVALID, "unsupported version: %d", version);
  Decoder D;
  D.s = In{(const uint8_t *)buf.data() + 8, (const uint8_t *)buf.data() + buf.size()};
  int64_t nl = 0;
  if (!D.read_int(nl)) return set_err(c, GN_ERR_INVALID, "failed to read layer count: %s", D.err.c_str());
  if (nl < INT32_MIN || nl > INT32_MAX) return set_err(c, GN_ERR_INVALID, "failed to read layer count: gob: value out of range");
  if (nl < 0 || nl > 1000) return set_err(c, GN_ERR_INVALID, "invalid number of layers: %lld (max 1000)", (long long)nl);
  std::string loss, opt;
  if (!D.read_string(loss)) return set_err(c, GN_ERR_INVALID, "failed to read loss type: %s", D.err.c_str());
  if (!D.read_string(opt)) return set_err(c, GN_ERR_INVALID, "failed to read optimizer type: %s", D.err.c_str());
  std::vector<LayerConfig> cfg((size_t)nl);
  int64_t total = 0;
  for (int64_t i = 0; i < nl; ++i) {
    if (!read_config(D, cfg[(size_t)i]))
      return set_err(c, GN_ERR_INVALID, "failed to read layer %lld: %s", (long long)i, D.err.c_str());
    total += (int64_t)cfg[(size_t)i].params.size();
  }
  const int64_t max_params = 256ll * 1024 * 1024;
  if (total > max_params)
    return set_err(c, GN_ERR_INVALID, "total parameters exceed limit: %lld (max %lld)", (long long)total,
                   (long long)max_params);
  std::vector<float> params;
  if (!D.read_floats(params)) return set_err(c, GN_ERR_INVALID, "failed to read parameters: %s", D.err.c_str());
  if ((int64_t)params.size() != total)
    return set_err(c, GN_ERR_INVALID, "parameter count mismatch: expected %lld, got %zu", (long long)total,
                   params.size());
  // CreateLayer
  std::vector<gn_layer_desc> ds((size_t)nl);
  for (int64_t i = 0; i < nl; ++i) {
    const LayerConfig &g = cfg[(size_t)i];
    gn_layer_desc &d = ds[(size_t)i];
    memset(&d, 0, sizeof d);
    d.in_channels = -1;
    int act = GN_ACT_RELU;
    if (g.type == "Dense" || g.type == "Conv2D") {
      act = activation_code(g.activation);
      if (act < 0)
        return set_err(c, GN_ERR_UNSUPPORTED, "layer %lld: activation %s is not built", (long long)i,
                       g.activation.c_str());
    }
    auto narrow = [](int64_t v) { return (int32_t)std::max<int64_t>(std::min<int64_t>(v, INT32_MAX), INT32_MIN); };
    if (g.type == "Dense") {
      d.kind = GN_LAYER_DENSE, d.in_size = narrow(g.in_size), d.out_size = narrow(g.out_size), d.act = act;
    } else if (g.type == "Conv2D") {
      d.kind = GN_LAYER_CONV2D, d.in_channels = narrow(g.in_channels), d.out_channels = narrow(g.out_channels);
      d.kernel = narrow(g.kernel), d.stride = narrow(g.stride), d.padding = narrow(g.padding), d.act = act;
    } else if (g.type == "Dropout") {
      d.kind = GN_LAYER_DROPOUT, d.p = g.prob, d.in_size = d.out_size = narrow(g.in_size);
    } else if (g.type == "BatchNorm2D") {
      d.kind = GN_LAYER_BATCHNORM2D, d.in_channels = narrow(g.in_channels), d.eps = g.eps, d.momentum = 0.1f;
      d.no_affine = !g.affine;
    } else if (g.type == "MaxPool2D" || g.type == "AvgPool2D") {
      d.kind = g.type == "MaxPool2D" ? GN_LAYER_MAXPOOL2D : GN_LAYER_AVGPOOL2D;
      d.in_channels = narrow(g.in_channels), d.kernel = narrow(g.kernel), d.stride = narrow(g.stride);
      d.padding = narrow(g.padding);
    } else if (g.type == "Embedding") {
      d.kind = GN_LAYER_EMBEDDING, d.vocab = narrow(g.in_size), d.dim = narrow(g.out_size);
    } else if (g.type == "Flatten") {
      d.kind = GN_LAYER_FLATTEN;
    } else if (g.type == "LayerNorm") {  // net.go:1544-1547: NewLayerNorm(NormalizedShape, Eps, Affine)
      if (!g.affine)
        return set_err(c, GN_ERR_UNSUPPORTED, "layer %lld: LayerNorm without affine parameters is not built",
                       (long long)i);
      d.kind = GN_LAYER_LAYERNORM, d.dim = narrow(g.normalized_shape), d.eps = g.eps;
    } else if (g.type == "LSTM" || g.type == "GRU" || g.type == "RBF") {
      return set_err(c, GN_ERR_UNSUPPORTED, "failed to create layer: %s is not built by this library",
                     g.type.c_str());
    } else {
      return set_err(c, GN_ERR_UNSUPPORTED, "failed to create layer: unsupported layer type: %s", g.type.c_str());
    }
    // the parameters of the layer the config describes (layer.go:267-300,
    // conv2d.go:74-130, batchnorm2d.go:70-135, embedding.go)
    int64_t want = 0;
    if (d.kind == GN_LAYER_DENSE) want = (int64_t)d.in_size * d.out_size + d.out_size;
    else if (d.kind == GN_LAYER_CONV2D)
      want = (int64_t)d.out_channels * d.in_channels * d.kernel * d.kernel + d.out_channels;
    else if (d.kind == GN_LAYER_BATCHNORM2D) want = d.no_affine ? 0 : 2 * (int64_t)d.in_channels;
    else if (d.kind == GN_LAYER_EMBEDDING) want = (int64_t)d.vocab * d.dim;
    else if (d.kind == GN_LAYER_LAYERNORM) want = 2 * (int64_t)d.dim;
    if (want != (int64_t)g.params.size())
      return set_err(c, GN_ERR_UNSUPPORTED,
                     "layer %lld (%s): the file holds %zu parameters, the layer its config describes %lld",
                     (long long)i, g.type.c_str(), g.params.size(), (long long)want);
  }
  // the first layer's input length: given, or what a Dense / Dropout config records
  if (nl > 0) {
    gn_layer_desc &d0 = ds[0];
    if (in_len > 0) {
      if (d0.kind != GN_LAYER_DENSE && d0.kind != GN_LAYER_DROPOUT) d0.in_size = in_len;
      else if (d0.in_size != in_len)
        return set_err(c, GN_ERR_SHAPE, "input length %d != the first layer's %d", in_len, d0.in_size);
    } else if (d0.kind != GN_LAYER_DENSE && d0.kind != GN_LAYER_DROPOUT) {
      return set_err(c, GN_ERR_INVALID, "a first %s layer needs the input length", cfg[0].type.c_str());
    }
  }
  int lk = GN_LOSS_MSE;  // net.go:966-976: anything else is MSE
  if (loss == "CrossEntropy") lk = GN_LOSS_CE;
  else if (loss == "Huber") return set_err(c, GN_ERR_UNSUPPORTED, "loss Huber is not built");
  if (opt != "Adam") return set_err(c, GN_ERR_UNSUPPORTED, "optimizer %s is not built (Adam only)", opt.c_str());
  const gn_adam_desc adam{0.001f, 0.9f, 0.999f, 1e-8f};  // opt.NewAdam(0.001), opt.go:117-126
  gn_model *M = nullptr;
  int rc = gn_model_create(c, ds.data(), (int32_t)nl, lk, &adam, max_batch, workers, &M);
  if (rc) return rc;
  int64_t off = 0;
  for (int64_t i = 0; i < nl && !rc; ++i) {
    int64_t o = 0, cnt = 0;
    rc = gn_model_layer_params(M, (int32_t)i, &o, &cnt);
    if (!rc && cnt != (int64_t)cfg[(size_t)i].params.size())
      rc = set_err(c, GN_ERR_INVALID, "layer %lld: %lld parameters built, %zu in the file", (long long)i,
                   (long long)cnt, cfg[(size_t)i].params.size());
    if (!rc && cnt) rc = gn_model_set_params(M, params.data() + off, o, cnt);
    off += cnt;
  }
  if (rc) {
    gn_model_destroy(M);
    return rc;
  }
  if (loss_kind) *loss_kind = lk;
  *out = M;
  return GN_OK;
}
