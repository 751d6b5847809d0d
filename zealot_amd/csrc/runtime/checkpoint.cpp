// checkpoint.cpp — ActorCritic::save / load (zealot-rl/src/ppo.rs:512-650) for
// the device-resident zl_ppo: a .safetensors image with the reference's
// tensor names and shapes, written and parsed here (host C++, no external
// library).
//
// safetensors layout: u64 little-endian header length N, N bytes of JSON
// {"name":{"dtype":"F32","shape":[..],"data_offsets":[begin,end]},...}
// padded with spaces to a multiple of 8, then the tensor bytes. Tensors are
// laid out sorted by dtype (descending in the format's dtype order: I64
// before F32) and then by name, which is the order the safetensors
// serializer uses, so a reference-layout checkpoint is byte-identical to the
// one the reference writes for the same values.
#include <cstdio>
#include <climits>
#include <cstring>
#include <map>
#include <memory>

#include "internal.hpp"

using namespace zl;

// A tensor name from an image, fit for an error message: bytes outside
// printable ASCII escaped as \xHH, at most 64 characters kept.
static std::string printable(const std::string& raw) {
  std::string out;
  for (size_t i = 0; i < raw.size() && out.size() < 64; ++i) {
    const unsigned char ch = (unsigned char)raw[i];
    if (ch >= 0x20 && ch < 0x7f) {
      out += (char)ch;
    } else {
      char b[5];
      snprintf(b, sizeof(b), "\\x%02x", ch);
      out += b;
    }
  }
  if (out.size() >= 64) out += "...";
  return out;
}

namespace {

enum Dt { DT_F32 = 0, DT_I64 = 1 };

struct Tensor {
  std::string name;
  Dt dt = DT_F32;
  std::vector<long long> shape;
  std::vector<unsigned char> bytes;
};

Tensor f32_tensor(std::string name, std::vector<long long> shape, const float* v) {
  Tensor t;
  t.name = std::move(name);
  t.shape = std::move(shape);
  long long n = 1;
  for (long long d : t.shape) n *= d;
  t.bytes.resize((size_t)n * 4);
  std::memcpy(t.bytes.data(), v, (size_t)n * 4);  // x86-64 and gfx950 are little-endian
  return t;
}

Tensor i64_tensor(std::string name, long long v) {
  Tensor t;
  t.name = std::move(name);
  t.dt = DT_I64;
  t.shape = {1};
  t.bytes.resize(8);
  std::memcpy(t.bytes.data(), &v, 8);
  return t;
}

std::vector<unsigned char> serialize(std::vector<Tensor>& ts) {
  std::sort(ts.begin(), ts.end(), [](const Tensor& a, const Tensor& b) {
    if (a.dt != b.dt) return a.dt > b.dt;  // I64 (8-byte) before F32
    return a.name < b.name;
  });
  std::string h = "{";
  size_t off = 0;
  for (size_t i = 0; i < ts.size(); ++i) {
    const Tensor& t = ts[i];
    if (i) h += ",";
    h += "\"" + t.name + "\":{\"dtype\":\"" + (t.dt == DT_F32 ? "F32" : "I64") + "\",\"shape\":[";
    for (size_t k = 0; k < t.shape.size(); ++k) h += (k ? "," : "") + std::to_string(t.shape[k]);
    h += "],\"data_offsets\":[" + std::to_string(off) + "," + std::to_string(off + t.bytes.size()) + "]}";
    off += t.bytes.size();
  }
  h += "}";
  while (h.size() % 8) h += ' ';
  std::vector<unsigned char> out(8 + h.size() + off);
  const unsigned long long n = h.size();
  std::memcpy(out.data(), &n, 8);
  std::memcpy(out.data() + 8, h.data(), h.size());
  size_t o = 8 + h.size();
  for (const Tensor& t : ts) {
    std::memcpy(out.data() + o, t.bytes.data(), t.bytes.size());
    o += t.bytes.size();
  }
  return out;
}

// ---- a small JSON reader for the header (objects, arrays, strings,
// non-negative integers; true / false / null and other numbers are accepted
// and skipped inside "__metadata__").
struct Json {
  enum Kind { OBJ, ARR, STR, NUM, OTHER } kind = OTHER;
  std::vector<std::pair<std::string, Json>> obj;
  std::vector<Json> arr;
  std::string str;
  long long num = -1;  // -1: not a non-negative integer
  const Json* get(const std::string& k) const {
    for (const auto& kv : obj)
      if (kv.first == k) return &kv.second;
    return nullptr;
  }
};

struct Parser {
  const char* p;
  const char* e;
  int depth = 0;
  void ws() {
    while (p < e && (*p == ' ' || *p == '\n' || *p == '\t' || *p == '\r')) ++p;
  }
  bool str(std::string* out) {
    if (p >= e || *p != '"') return false;
    ++p;
    while (p < e && *p != '"') {
      if (*p == '\\') {
        if (++p >= e) return false;
        switch (*p) {
          case '"': case '\\': case '/': out->push_back(*p); break;
          case 'n': out->push_back('\n'); break;
          case 't': out->push_back('\t'); break;
          case 'r': out->push_back('\r'); break;
          case 'b': out->push_back('\b'); break;
          case 'f': out->push_back('\f'); break;
          case 'u':  // kept as written: names here are ASCII
            if (e - p < 5) return false;
            out->append(p - 1, 6);
            p += 4;
            break;
          default: return false;
        }
        ++p;
      } else {
        out->push_back(*p++);
      }
    }
    if (p >= e) return false;
    ++p;
    return true;
  }
  bool value(Json* v) {
    if (++depth > 16) return false;
    ws();
    if (p >= e) return false;
    bool ok = true;
    if (*p == '{') {
      v->kind = Json::OBJ;
      ++p;
      ws();
      if (p < e && *p == '}') {
        ++p;
      } else {
        while (ok) {
          ws();
          std::string k;
          if (!str(&k)) return false;
          ws();
          if (p >= e || *p != ':') return false;
          ++p;
          Json c;
          if (!value(&c)) return false;
          v->obj.emplace_back(std::move(k), std::move(c));
          ws();
          if (p < e && *p == ',') { ++p; continue; }
          if (p < e && *p == '}') { ++p; break; }
          return false;
        }
      }
    } else if (*p == '[') {
      v->kind = Json::ARR;
      ++p;
      ws();
      if (p < e && *p == ']') {
        ++p;
      } else {
        while (true) {
          Json c;
          if (!value(&c)) return false;
          v->arr.push_back(std::move(c));
          ws();
          if (p < e && *p == ',') { ++p; continue; }
          if (p < e && *p == ']') { ++p; break; }
          return false;
        }
      }
    } else if (*p == '"') {
      v->kind = Json::STR;
      ok = str(&v->str);
    } else if (*p >= '0' && *p <= '9') {
      v->kind = Json::NUM;
      long long n = 0;
      while (p < e && *p >= '0' && *p <= '9') {
        if (n > (1LL << 56)) return false;
        n = n * 10 + (*p++ - '0');
      }
      v->num = n;
      if (p < e && (*p == '.' || *p == 'e' || *p == 'E')) {  // not an integer
        v->num = -1;
        while (p < e && (strchr("0123456789.eE+-", *p))) ++p;
      }
    } else {
      // true / false / null / negative numbers (only legal in metadata)
      v->kind = Json::OTHER;
      const char* s = p;
      while (p < e && strchr("truefalsn-0123456789.eE+", *p)) ++p;
      ok = p > s;
    }
    --depth;
    return ok;
  }
};

struct Entry {
  Dt dt;
  std::vector<long long> shape;
  const unsigned char* data;
  size_t nbytes;
};

// Parse and validate a safetensors image: every tensor's byte range lies in
// the data section, matches its dtype and shape, and the ranges tile the
// data section without gaps or overlap (the format's own rule).
zl_status parse(zl_ctx* c, const unsigned char* buf, size_t size, std::map<std::string, Entry>* out) {
  if (size < 8) return fail(c, ZL_ERR_INVALID, "checkpoint: %zu bytes, no header", size);
  unsigned long long n = 0;
  std::memcpy(&n, buf, 8);
  if (n > size - 8 || n > (1ULL << 27))
    return fail(c, ZL_ERR_INVALID, "checkpoint: header length %llu beyond the image", n);
  Parser ps{(const char*)buf + 8, (const char*)buf + 8 + n};
  Json root;
  if (!ps.value(&root) || root.kind != Json::OBJ)
    return fail(c, ZL_ERR_INVALID, "checkpoint: header is not a JSON object");
  ps.ws();
  if (ps.p != ps.e) return fail(c, ZL_ERR_INVALID, "checkpoint: trailing bytes after the header");
  const unsigned char* data = buf + 8 + n;
  const size_t dsize = size - 8 - n;
  std::vector<std::pair<size_t, size_t>> ranges;
  for (const auto& kv : root.obj) {
    if (kv.first == "__metadata__") continue;
    const Json& t = kv.second;
    const Json* dt = t.get("dtype");
    const Json* sh = t.get("shape");
    const Json* of = t.get("data_offsets");
    if (t.kind != Json::OBJ || !dt || dt->kind != Json::STR || !sh || sh->kind != Json::ARR || !of ||
        of->kind != Json::ARR || of->arr.size() != 2 || of->arr[0].num < 0 || of->arr[1].num < 0)
      return fail(c, ZL_ERR_INVALID, "checkpoint: malformed entry '%s'", printable(kv.first).c_str());
    size_t esize = 0;
    Entry en{};
    if (dt->str == "F32") {
      en.dt = DT_F32;
      esize = 4;
    } else if (dt->str == "I64") {
      en.dt = DT_I64;
      esize = 8;
    } else {
      en.dt = DT_F32;
      esize = 0;  // another dtype: its range still counts, the tensor is unusable here
    }
    long long count = 1;
    for (const Json& d : sh->arr) {
      if (d.num < 0 || (d.num > 0 && count > (1LL << 40) / d.num))
        return fail(c, ZL_ERR_INVALID, "checkpoint: bad shape of '%s'", printable(kv.first).c_str());
      en.shape.push_back(d.num);
      count *= d.num;
    }
    const size_t b = (size_t)of->arr[0].num, e = (size_t)of->arr[1].num;
    if (b > e || e > dsize || (esize && (e - b) != (size_t)count * esize))
      return fail(c, ZL_ERR_INVALID, "checkpoint: data offsets of '%s' do not match its shape",
                  printable(kv.first).c_str());
    ranges.emplace_back(b, e);
    if (esize) {
      en.data = data + b;
      en.nbytes = e - b;
      (*out)[kv.first] = en;
    }
  }
  std::sort(ranges.begin(), ranges.end());
  size_t at = 0;
  for (const auto& r : ranges) {
    if (r.first != at) return fail(c, ZL_ERR_INVALID, "checkpoint: tensor data overlaps or has gaps");
    at = r.second;
  }
  if (at != dsize) return fail(c, ZL_ERR_INVALID, "checkpoint: %zu unused data bytes", dsize - at);
  return ZL_OK;
}

// The Mlp under `prefix` (ppo.rs:585-610): layers w_0, b_0, w_1, ... while
// present; dims from the weight shapes [out, in].
zl_status read_mlp(zl_ctx* c, const std::map<std::string, Entry>& m, const std::string& prefix,
                   std::vector<int>* dims, std::vector<const Entry*>* ws,
                   std::vector<const Entry*>* bs) {
  dims->clear();
  for (int l = 0;; ++l) {
    auto w = m.find(prefix + ".w_" + std::to_string(l));
    if (w == m.end()) break;
    auto b = m.find(prefix + ".b_" + std::to_string(l));
    if (b == m.end())
      return fail(c, ZL_ERR_INVALID, "checkpoint: %s.b_%d missing", prefix.c_str(), l);
    const Entry& we = w->second;
    if (we.dt != DT_F32 || we.shape.size() != 2 || b->second.dt != DT_F32 ||
        b->second.shape.size() != 1 || b->second.shape[0] != we.shape[0] || we.shape[0] > (1 << 30) ||
        we.shape[1] > (1 << 30))
      return fail(c, ZL_ERR_INVALID, "checkpoint: %s layer %d: expected F32 w [out, in], b [out]",
                  prefix.c_str(), l);
    if (l == 0) dims->push_back((int)we.shape[1]);
    else if ((int)we.shape[1] != dims->back())
      return fail(c, ZL_ERR_INVALID, "checkpoint: %s layer %d input %lld != previous output %d",
                  prefix.c_str(), l, we.shape[1], dims->back());
    dims->push_back((int)we.shape[0]);
    ws->push_back(&we);
    bs->push_back(&b->second);
  }
  if (ws->empty()) return fail(c, ZL_ERR_INVALID, "checkpoint: no layers under prefix `%s`", prefix.c_str());
  return ZL_OK;
}

zl_status read_vec(zl_ctx* c, const std::map<std::string, Entry>& m, const std::string& name,
                   size_t n, std::vector<float>* out) {
  auto it = m.find(name);
  if (it == m.end()) return fail(c, ZL_ERR_INVALID, "checkpoint: tensor '%s' missing", name.c_str());
  if (it->second.dt != DT_F32 || it->second.nbytes != n * 4)
    return fail(c, ZL_ERR_INVALID, "checkpoint: '%s' is not F32 [%zu]", name.c_str(), n);
  out->resize(n);
  std::memcpy(out->data(), it->second.data, n * 4);
  return ZL_OK;
}

long long packed_count(const std::vector<int>& d) {
  long long n = 0;
  for (size_t l = 0; l + 1 < d.size(); ++l) n += (long long)d[l + 1] * d[l] + d[l + 1];
  return n;
}

// Append per-layer tensors "<prefix>.w_l" / "<prefix>.b_l" from a packed net.
void add_net(std::vector<Tensor>* ts, const std::string& prefix, const std::vector<int>& d,
             const float* packed) {
  for (size_t l = 0; l + 1 < d.size(); ++l) {
    const int in = d[l], out = d[l + 1];
    ts->push_back(f32_tensor(prefix + ".w_" + std::to_string(l), {out, in}, packed));
    packed += (size_t)out * in;
    ts->push_back(f32_tensor(prefix + ".b_" + std::to_string(l), {out}, packed));
    packed += out;
  }
}

// Inverse of add_net into a packed buffer.
void get_net(const std::vector<const Entry*>& ws, const std::vector<const Entry*>& bs, float* packed) {
  for (size_t l = 0; l < ws.size(); ++l) {
    std::memcpy(packed, ws[l]->data, ws[l]->nbytes);
    packed += ws[l]->nbytes / 4;
    std::memcpy(packed, bs[l]->data, bs[l]->nbytes);
    packed += bs[l]->nbytes / 4;
  }
}

zl_status build_image(zl_ppo* p, const float* obs_norm, const float* critic_norm, int with_opt,
                      std::vector<unsigned char>* img) {
  zl_ctx* c = ppo_ctx(p);
  std::vector<int> ad, cd;
  ppo_dims(p, &ad, &cd);
  const int A = ad.back(), od = ad[0], cdim = cd[0];
  std::vector<float> actor((size_t)packed_count(ad)), critic((size_t)packed_count(cd)), ls(A);
  float lr = 0.0f;
  zl_status s = zl_ppo_get_params(p, actor.data(), critic.data(), ls.data(), &lr);
  if (s) return s;
  // Normaliser states (a NULL state is saved as Normalizer::new).
  auto norm = [&](const float* dev, int dim, std::vector<float>* st) -> zl_status {
    st->assign((size_t)2 * dim + 1, 0.0f);
    if (!dev) {
      for (int i = dim; i <= 2 * dim; ++i) (*st)[i] = 1.0f;
      return ZL_OK;
    }
    ZL_HIP(c, hipMemcpyAsync(st->data(), dev, st->size() * 4, hipMemcpyDeviceToHost, c->stream));
    ZL_HIP(c, hipStreamSynchronize(c->stream));
    return ZL_OK;
  };
  std::vector<float> on, cn;
  if ((s = norm(obs_norm, od, &on)) || (s = norm(critic_norm, cdim, &cn))) return s;
  std::vector<Tensor> ts;
  add_net(&ts, "actor", ad, actor.data());
  add_net(&ts, "critic", cd, critic.data());
  ts.push_back(f32_tensor("log_std", {A}, ls.data()));
  ts.push_back(f32_tensor("obs_norm.mean", {od}, on.data()));
  ts.push_back(f32_tensor("obs_norm.m2", {od}, on.data() + od));
  ts.push_back(f32_tensor("obs_norm.count", {1}, on.data() + 2 * od));
  ts.push_back(f32_tensor("critic_norm.mean", {cdim}, cn.data()));
  ts.push_back(f32_tensor("critic_norm.m2", {cdim}, cn.data() + cdim));
  ts.push_back(f32_tensor("critic_norm.count", {1}, cn.data() + 2 * cdim));
  ts.push_back(f32_tensor("lr", {1}, &lr));
  if (with_opt) {
    std::vector<float> ma(actor.size()), va(actor.size()), mc(critic.size()), vc(critic.size()),
        mls(A), vls(A);
    if ((s = zl_ppo_get_moments(p, ma.data(), va.data(), mc.data(), vc.data(), mls.data(), vls.data())))
      return s;
    int t = 0;
    unsigned long long gstep = 0;
    zl_ppo_get_counters(p, &t, &gstep);
    add_net(&ts, "adam_m.actor", ad, ma.data());
    add_net(&ts, "adam_v.actor", ad, va.data());
    add_net(&ts, "adam_m.critic", cd, mc.data());
    add_net(&ts, "adam_v.critic", cd, vc.data());
    ts.push_back(f32_tensor("adam_m.log_std", {A}, mls.data()));
    ts.push_back(f32_tensor("adam_v.log_std", {A}, vls.data()));
    ts.push_back(i64_tensor("adam.t", t));
    ts.push_back(i64_tensor("adam.gstep", (long long)gstep));
  }
  *img = serialize(ts);
  return ZL_OK;
}

zl_status load_image(zl_ppo* p, float* obs_norm, float* critic_norm, int restore_opt,
                     const unsigned char* buf, size_t size) {
  zl_ctx* c = ppo_ctx(p);
  std::map<std::string, Entry> m;
  zl_status s = parse(c, buf, size, &m);
  if (s) return s;
  std::vector<int> ad, cd, fad, fcd;
  ppo_dims(p, &ad, &cd);
  std::vector<const Entry*> aw, ab, cw, cb;
  if ((s = read_mlp(c, m, "actor", &fad, &aw, &ab)) || (s = read_mlp(c, m, "critic", &fcd, &cw, &cb)))
    return s;
  if (fad != ad || fcd != cd)
    return fail(c, ZL_ERR_INVALID, "checkpoint: net dims differ from this handle's");
  const int A = ad.back(), od = ad[0], cdim = cd[0];
  std::vector<float> ls, on_m, on_q, on_n, cn_m, cn_q, cn_n, lr;
  if ((s = read_vec(c, m, "log_std", A, &ls)) || (s = read_vec(c, m, "obs_norm.mean", od, &on_m)) ||
      (s = read_vec(c, m, "obs_norm.m2", od, &on_q)) || (s = read_vec(c, m, "obs_norm.count", 1, &on_n)) ||
      (s = read_vec(c, m, "critic_norm.mean", cdim, &cn_m)) ||
      (s = read_vec(c, m, "critic_norm.m2", cdim, &cn_q)) ||
      (s = read_vec(c, m, "critic_norm.count", 1, &cn_n)) || (s = read_vec(c, m, "lr", 1, &lr)))
    return s;
  // Optional optimizer state: all of it or none.
  bool have_opt = restore_opt && m.count("adam.t") && m.count("adam.gstep");
  std::vector<float> ma, va, mc, vc, mls, vls;
  long long opt_t = 0, opt_gstep = 0;
  if (have_opt) {
    std::vector<int> d;
    std::vector<const Entry*> w[4], b[4];
    const char* pre[4] = {"adam_m.actor", "adam_v.actor", "adam_m.critic", "adam_v.critic"};
    std::vector<float>* dst[4] = {&ma, &va, &mc, &vc};
    for (int i = 0; i < 4; ++i) {
      if ((s = read_mlp(c, m, pre[i], &d, &w[i], &b[i]))) return s;
      if (d != (i < 2 ? ad : cd)) return fail(c, ZL_ERR_INVALID, "checkpoint: %s dims differ", pre[i]);
      dst[i]->resize((size_t)packed_count(d));
      get_net(w[i], b[i], dst[i]->data());
    }
    if ((s = read_vec(c, m, "adam_m.log_std", A, &mls)) || (s = read_vec(c, m, "adam_v.log_std", A, &vls)))
      return s;
    const Entry& et = m.at("adam.t");
    const Entry& eg = m.at("adam.gstep");
    if (et.dt != DT_I64 || et.nbytes != 8 || eg.dt != DT_I64 || eg.nbytes != 8)
      return fail(c, ZL_ERR_INVALID, "checkpoint: adam counters are not I64 [1]");
    std::memcpy(&opt_t, et.data, 8);
    std::memcpy(&opt_gstep, eg.data, 8);
    // The step count feeds powi(beta, t) (an i32 exponent) and gstep the
    // trainer's bias correction: out-of-range values are a corrupt image.
    if (opt_t < 0 || opt_t > INT_MAX || opt_gstep < 0)
      return fail(c, ZL_ERR_INVALID, "checkpoint: adam counters out of range (t %lld, gstep %lld)",
                  opt_t, opt_gstep);
  }
  std::vector<float> actor((size_t)packed_count(ad)), critic((size_t)packed_count(cd));
  get_net(aw, ab, actor.data());
  get_net(cw, cb, critic.data());
  if ((s = zl_ppo_set_params(p, actor.data(), critic.data(), ls.data(), lr[0]))) return s;
  if (have_opt) {
    if ((s = ppo_set_moments(p, ma.data(), va.data(), mc.data(), vc.data(), mls.data(), vls.data())))
      return s;
    ppo_set_counters(p, (int)opt_t, (unsigned long long)opt_gstep);
  } else if ((s = zl_ppo_reset_optimizer(p))) {  // ppo.rs:625-636: fresh Adam state
    return s;
  }
  auto put = [&](float* dev, int dim, const std::vector<float>& mean, const std::vector<float>& m2,
                 float count) -> zl_status {
    if (!dev) return ZL_OK;
    std::vector<float> st((size_t)2 * dim + 1);
    std::memcpy(st.data(), mean.data(), (size_t)dim * 4);
    std::memcpy(st.data() + dim, m2.data(), (size_t)dim * 4);
    st[2 * dim] = count;
    ZL_HIP(c, hipMemcpyAsync(dev, st.data(), st.size() * 4, hipMemcpyHostToDevice, c->stream));
    ZL_HIP(c, hipStreamSynchronize(c->stream));
    return ZL_OK;
  };
  if ((s = put(obs_norm, od, on_m, on_q, on_n[0])) || (s = put(critic_norm, cdim, cn_m, cn_q, cn_n[0])))
    return s;
  return ZL_OK;
}

}  // namespace

extern "C" {

zl_status zl_ppo_save_bytes(zl_ppo* p, const float* obs_norm, const float* critic_norm,
                            int with_optimizer, void* buf, size_t cap, size_t* size) {
  if (!p) return ZL_ERR_INVALID;
  if (!size) return fail(ppo_ctx(p), ZL_ERR_INVALID, "zl_ppo_save_bytes: null size");
  std::vector<unsigned char> img;
  zl_status s = build_image(p, obs_norm, critic_norm, with_optimizer, &img);
  if (s) return s;
  *size = img.size();
  if (!buf) return ZL_OK;
  if (cap < img.size())
    return fail(ppo_ctx(p), ZL_ERR_INVALID, "zl_ppo_save_bytes: buffer of %zu bytes < %zu", cap,
                img.size());
  std::memcpy(buf, img.data(), img.size());
  return ZL_OK;
}

zl_status zl_ppo_save(zl_ppo* p, const float* obs_norm, const float* critic_norm, int with_optimizer,
                      const char* path) {
  if (!p) return ZL_ERR_INVALID;
  zl_ctx* c = ppo_ctx(p);
  if (!path) return fail(c, ZL_ERR_INVALID, "zl_ppo_save: null path");
  std::vector<unsigned char> img;
  zl_status s = build_image(p, obs_norm, critic_norm, with_optimizer, &img);
  if (s) return s;
  FILE* f = fopen(path, "wb");
  if (!f) return fail(c, ZL_ERR_INVALID, "zl_ppo_save: cannot open %s", path);
  const size_t w = fwrite(img.data(), 1, img.size(), f);
  const int cl = fclose(f);
  if (w != img.size() || cl != 0) return fail(c, ZL_ERR_INVALID, "zl_ppo_save: short write to %s", path);
  return ZL_OK;
}

zl_status zl_ppo_load_bytes(zl_ppo* p, float* obs_norm, float* critic_norm, int restore_optimizer,
                            const void* buf, size_t size) {
  if (!p) return ZL_ERR_INVALID;
  if (!buf) return fail(ppo_ctx(p), ZL_ERR_INVALID, "zl_ppo_load_bytes: null buffer");
  return load_image(p, obs_norm, critic_norm, restore_optimizer, (const unsigned char*)buf, size);
}

zl_status zl_ppo_load(zl_ppo* p, float* obs_norm, float* critic_norm, int restore_optimizer,
                      const char* path) {
  if (!p) return ZL_ERR_INVALID;
  zl_ctx* c = ppo_ctx(p);
  if (!path) return fail(c, ZL_ERR_INVALID, "zl_ppo_load: null path");
  FILE* f = fopen(path, "rb");
  if (!f) return fail(c, ZL_ERR_INVALID, "zl_ppo_load: cannot open %s", path);
  std::vector<unsigned char> img;
  unsigned char chunk[1 << 16];
  size_t r;
  while ((r = fread(chunk, 1, sizeof(chunk), f)) > 0) img.insert(img.end(), chunk, chunk + r);
  const bool err = ferror(f) != 0;
  fclose(f);
  if (err) return fail(c, ZL_ERR_INVALID, "zl_ppo_load: read error on %s", path);
  return load_image(p, obs_norm, critic_norm, restore_optimizer, img.data(), img.size());
}

zl_status zl_checkpoint_dims(const void* buf, size_t size, int* actor_dims, int* n_actor,
                             int* critic_dims, int* n_critic, int cap) {
  if (!buf || !n_actor || !n_critic) return fail(nullptr, ZL_ERR_INVALID, "zl_checkpoint_dims: null argument");
  std::map<std::string, Entry> m;
  zl_status s = parse(nullptr, (const unsigned char*)buf, size, &m);
  if (s) return s;
  std::vector<int> ad, cd;
  std::vector<const Entry*> w, b;
  if ((s = read_mlp(nullptr, m, "actor", &ad, &w, &b))) return s;
  w.clear();
  b.clear();
  if ((s = read_mlp(nullptr, m, "critic", &cd, &w, &b))) return s;
  *n_actor = (int)ad.size();
  *n_critic = (int)cd.size();
  if ((int)ad.size() > cap || (int)cd.size() > cap)
    return fail(nullptr, ZL_ERR_INVALID, "zl_checkpoint_dims: %zu / %zu dims > capacity %d", ad.size(),
                cd.size(), cap);
  if (actor_dims) std::copy(ad.begin(), ad.end(), actor_dims);
  if (critic_dims) std::copy(cd.begin(), cd.end(), critic_dims);
  return ZL_OK;
}

}  // extern "C"
