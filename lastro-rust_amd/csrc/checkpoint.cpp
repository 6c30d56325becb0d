// Checkpoint loading on the host: the safetensors index and BF16 tensor reader (Checkpoint::open / bf16,
// rust/moe-rt/src/weights.rs:52-122), the Granite config.json (Config::from_json, rust/moe-rt/src/model.rs:34-61) and
// the host model (HostModel::load, model.rs:100-132; HostLayer::load, block.rs:31-53) with each BF16 matrix quantised
// on load to the engine's Q8_0 / Q4_0 blocks (or kept f32), so that the result can be handed to moert_model_create.
//
// safetensors: 8 bytes little-endian header length n, then n bytes of JSON {name: {dtype, shape, data_offsets}} (plus
// an optional "__metadata__"), then the data; offsets are relative to byte 8 + n. Only the index stays in memory;
// every tensor is read from its file with a positional read when asked for.
#include <dirent.h>
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "../../include/moert.h"
#include "host_utils.h"
#include "json.h"

namespace moert {
int set_error(int code, const char* fmt, ...);
}

using moert::set_error;
using moert::JParser;
using moert::JVal;

namespace {

// ---- safetensors ------------------------------------------------------------------------------------------------
struct Entry {
  int file;
  std::string dtype;
  std::vector<uint64_t> shape;
  uint64_t start, end;
};

constexpr uint64_t kMaxHeader = (uint64_t)100 << 20;

bool read_at(int fd, void* dst, size_t n, uint64_t off) {
  uint8_t* d = (uint8_t*)dst;
  while (n > 0) {
    const ssize_t r = pread(fd, d, n, (off_t)off);
    if (r <= 0) return false;
    d += r;
    n -= (size_t)r;
    off += (uint64_t)r;
  }
  return true;
}

}  // namespace

struct moert_checkpoint {
  std::vector<std::pair<std::string, int>> files;  // path, descriptor
  std::map<std::string, Entry> index;
  ~moert_checkpoint() {
    for (auto& f : files)
      if (f.second >= 0) close(f.second);
  }
};

struct moert_host_model {
  moert_config cfg{};
  int wdtype = 0, embed_dtype = 0;
  std::vector<std::vector<uint8_t>> blobs;  // quantised matrices
  std::vector<std::vector<float>> f32s;     // norm weights
  std::vector<moert_layer_weights> layers;
  moert_model_weights w{};
};

namespace {

int open_file(moert_checkpoint* ck, const std::string& path) {
  const int fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0) return set_error(MOERT_E_CONFIG, "safetensors: cannot open %s", path.c_str());
  const int fi = (int)ck->files.size();
  ck->files.push_back({path, fd});
  struct stat st;
  if (fstat(fd, &st) != 0) return set_error(MOERT_E_CONFIG, "safetensors: cannot stat %s", path.c_str());
  const uint64_t size = (uint64_t)st.st_size;
  uint8_t lb[8];
  if (!read_at(fd, lb, 8, 0)) return set_error(MOERT_E_CONFIG, "safetensors: %s shorter than 8 bytes", path.c_str());
  uint64_t n = 0;
  for (int i = 7; i >= 0; i--) n = (n << 8) | lb[i];
  if (n > kMaxHeader) return set_error(MOERT_E_CONFIG, "safetensors: header of %llu bytes in %s",
                                       (unsigned long long)n, path.c_str());
  if (n > size - 8) return set_error(MOERT_E_CONFIG, "safetensors: header past the end of %s", path.c_str());
  std::vector<char> head(n);
  if (!read_at(fd, head.data(), n, 8)) return set_error(MOERT_E_CONFIG, "safetensors: short read of %s", path.c_str());
  JVal j;
  std::string err;
  if (!JParser(head.data(), n).parse(j, err)) return set_error(MOERT_E_CONFIG, "safetensors: %s", err.c_str());
  if (j.kind != JVal::OBJ) return set_error(MOERT_E_CONFIG, "safetensors: header is not an object");
  for (const auto& kv : j.obj) {
    const std::string& name = kv.first;
    if (name == "__metadata__") continue;
    const JVal& v = kv.second;
    const JVal* dt = v.get("dtype");
    if (!dt || dt->kind != JVal::STR) return set_error(MOERT_E_CONFIG, "safetensors: %s: no dtype", name.c_str());
    const JVal* sh = v.get("shape");
    if (!sh || sh->kind != JVal::ARR) return set_error(MOERT_E_CONFIG, "safetensors: %s: no shape", name.c_str());
    Entry e{fi, dt->s, {}, 0, 0};
    for (const JVal& d : sh->arr) {
      if (d.kind != JVal::NUM || !d.is_uint) return set_error(MOERT_E_CONFIG, "safetensors: %s: bad shape", name.c_str());
      e.shape.push_back(d.u);
    }
    const JVal* off = v.get("data_offsets");
    if (!off || off->kind != JVal::ARR)
      return set_error(MOERT_E_CONFIG, "safetensors: %s: no data_offsets", name.c_str());
    if (off->arr.size() != 2)
      return set_error(MOERT_E_CONFIG, "safetensors: %s: data_offsets must be [begin, end], got %zu numbers", name.c_str(),
                       off->arr.size());
    const JVal &a = off->arr[0], &b = off->arr[1];
    if (a.kind != JVal::NUM || !a.is_uint || b.kind != JVal::NUM || !b.is_uint)
      return set_error(MOERT_E_CONFIG, "safetensors: %s: data_offsets not numeric", name.c_str());
    const uint64_t base = 8 + n;
    if (a.u > UINT64_MAX - base || b.u > UINT64_MAX - base || a.u > b.u || base + b.u > size)
      return set_error(MOERT_E_CONFIG, "safetensors: %s: the tensor's byte range ends past the data section", name.c_str());
    e.start = base + a.u;
    e.end = base + b.u;
    ck->index[name] = std::move(e);
  }
  return MOERT_OK;
}

// Product of the shape times `elem` bytes, or false on overflow.
bool shape_bytes(const std::vector<uint64_t>& shape, uint64_t elem, uint64_t* out) {
  uint64_t b = elem;
  for (uint64_t d : shape) {
    if (d != 0 && b > UINT64_MAX / d) return false;
    b *= d;
  }
  *out = b;
  return true;
}

int read_bf16(const moert_checkpoint* ck, const char* name, std::vector<uint16_t>& out,
              std::vector<uint64_t>* shape_out) {
  auto it = ck->index.find(name);
  if (it == ck->index.end()) return set_error(MOERT_E_CONFIG, "safetensors: tensor missing: %s", name);
  const Entry& e = it->second;
  if (e.dtype != "BF16")
    return set_error(MOERT_E_CONFIG, "safetensors: %s: dtype %s (expected BF16)", name, e.dtype.c_str());
  uint64_t bytes = 0;
  if (!shape_bytes(e.shape, 2, &bytes) || bytes != e.end - e.start)
    return set_error(MOERT_E_CONFIG, "safetensors: %s: byte count differs from dtype size x product of the shape", name);
  out.resize(bytes / 2);
  if (!read_at(ck->files[e.file].second, out.data(), bytes, e.start))
    return set_error(MOERT_E_CONFIG, "safetensors: %s: short read", name);
  if (shape_out) *shape_out = e.shape;
  return MOERT_OK;
}

inline float bf16_to_f32(uint16_t b) {
  const uint32_t u = (uint32_t)b << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// A BF16 tensor of exactly `shape`, widened to f32 (exact).
int read_f32(const moert_checkpoint* ck, const std::string& name, const std::vector<uint64_t>& shape,
             std::vector<float>& out) {
  std::vector<uint16_t> raw;
  std::vector<uint64_t> s;
  int rc = read_bf16(ck, name.c_str(), raw, &s);
  if (rc) return rc;
  if (s != shape) {
    std::string want, got;
    for (uint64_t d : shape) want += std::to_string(d) + ",";
    for (uint64_t d : s) got += std::to_string(d) + ",";
    return set_error(MOERT_E_CONFIG, "safetensors: %s: shape [%s] (expected [%s])", name.c_str(), got.c_str(),
                     want.c_str());
  }
  out.resize(raw.size());
  moert::parallel_for(raw.size(), 1 << 16, [&](size_t a, size_t b) {
    for (size_t i = a; i < b; i++) out[i] = bf16_to_f32(raw[i]);
  });
  return MOERT_OK;
}

// A BF16 matrix quantised to `dtype` (Q8_0 / Q4_0 blocks along rows, or f32).
int read_matrix(const moert_checkpoint* ck, const std::string& name, const std::vector<uint64_t>& shape, int dtype,
                std::vector<uint8_t>& out) {
  std::vector<float> f;
  int rc = read_f32(ck, name, shape, f);
  if (rc) return rc;
  if (shape.back() % 32) return set_error(MOERT_E_CONFIG, "%s: rows of %llu, not a multiple of 32", name.c_str(),
                                          (unsigned long long)shape.back());
  out.resize(moert::dtype_bytes(dtype, f.size()));
  const size_t bb = moert::dtype_bytes(dtype, 32);
  moert::parallel_for(f.size() / 32, 4096, [&](size_t a, size_t b) {
    moert::quantize(f.data() + a * 32, (b - a) * 32, dtype, out.data() + a * bb);
  });
  return MOERT_OK;
}

}  // namespace

extern "C" {

int moert_config_from_json(const char* json, size_t len, moert_config* out) {
  if (!json || !out) return set_error(MOERT_E_CONFIG, "config: null argument");
  JVal v;
  std::string err;
  if (!JParser(json, len).parse(v, err)) return set_error(MOERT_E_CONFIG, "config.json: %s", err.c_str());
  if (v.kind != JVal::OBJ) return set_error(MOERT_E_CONFIG, "config.json is not an object");
  const JVal* mt = v.get("model_type");
  if (!mt || mt->kind != JVal::STR || mt->s != "granitemoe")
    return set_error(MOERT_E_CONFIG, "config.json: model_type %s (expected granitemoe)",
                     mt && mt->kind == JVal::STR ? mt->s.c_str() : "missing");
  const JVal* rs = v.get("rope_scaling");
  const JVal* ab = v.get("attention_bias");
  const JVal* tie = v.get("tie_word_embeddings");
  if ((rs && rs->kind != JVal::NUL) || (ab && ab->kind == JVal::BOOL && ab->b) ||
      (tie && tie->kind == JVal::BOOL && !tie->b))
    return set_error(MOERT_E_CONFIG, "config.json: unsupported variant (rope_scaling, attention_bias or untied "
                                     "embeddings)");
  moert_config c{};
  auto u = [&](const char* k, int* dst) -> bool {
    const JVal* x = v.get(k);
    if (!x || x->kind != JVal::NUM || !x->is_uint || x->u > 1u << 30) return false;
    *dst = (int)x->u;
    return true;
  };
  auto f = [&](const char* k, float* dst) -> bool {
    const JVal* x = v.get(k);
    if (!x || x->kind != JVal::NUM) return false;
    *dst = (float)x->num;
    return true;
  };
  const char* ints[] = {"hidden_size", "intermediate_size", "num_hidden_layers", "num_attention_heads",
                        "num_key_value_heads", "vocab_size", "num_local_experts", "num_experts_per_tok"};
  int* dsti[] = {&c.hidden, &c.inter, &c.layers, &c.heads, &c.kv_heads, &c.vocab, &c.experts, &c.top_k};
  for (int i = 0; i < 8; i++)
    if (!u(ints[i], dsti[i])) return set_error(MOERT_E_CONFIG, "config.json: no %s", ints[i]);
  const char* flts[] = {"rope_theta", "rms_norm_eps", "embedding_multiplier", "residual_multiplier",
                        "attention_multiplier", "logits_scaling"};
  float* dstf[] = {&c.rope_theta, &c.eps, &c.embedding_multiplier, &c.residual_multiplier, &c.attention_multiplier,
                   &c.logits_scaling};
  for (int i = 0; i < 6; i++)
    if (!f(flts[i], dstf[i])) return set_error(MOERT_E_CONFIG, "config.json: no %s", flts[i]);
  const JVal* hd = v.get("head_dim");
  if (hd && hd->kind == JVal::NUM && hd->is_uint)
    c.head_dim = (int)hd->u;
  else if (c.heads > 0)
    c.head_dim = c.hidden / c.heads;
  else
    return set_error(MOERT_E_CONFIG, "config.json: num_attention_heads is 0");
  *out = c;
  return MOERT_OK;
}

int moert_checkpoint_open(const char* dir, moert_checkpoint** out) {
  if (!dir || !out) return set_error(MOERT_E_CONFIG, "checkpoint: null argument");
  *out = nullptr;
  DIR* d = opendir(dir);
  if (!d) return set_error(MOERT_E_CONFIG, "checkpoint: cannot read directory %s", dir);
  std::vector<std::string> paths;
  while (dirent* e = readdir(d)) {
    const std::string n = e->d_name;
    if (n.size() > 12 && n.compare(n.size() - 12, 12, ".safetensors") == 0) paths.push_back(std::string(dir) + "/" + n);
  }
  closedir(d);
  std::sort(paths.begin(), paths.end());
  if (paths.empty()) return set_error(MOERT_E_CONFIG, "checkpoint: no *.safetensors in %s", dir);
  std::unique_ptr<moert_checkpoint> ck(new moert_checkpoint);
  for (const std::string& p : paths) {
    const int rc = open_file(ck.get(), p);
    if (rc) return rc;
  }
  *out = ck.release();
  return MOERT_OK;
}

int moert_checkpoint_close(moert_checkpoint* ck) {
  delete ck;
  return MOERT_OK;
}

int moert_checkpoint_tensor(const moert_checkpoint* ck, const char* name, char* dtype, int dtype_len,
                            uint64_t* shape, int max_dims, int* ndim) {
  if (!ck || !name) return set_error(MOERT_E_CONFIG, "checkpoint: null argument");
  auto it = ck->index.find(name);
  if (it == ck->index.end()) return set_error(MOERT_E_RANGE, "safetensors: tensor missing: %s", name);
  const Entry& e = it->second;
  if (dtype && dtype_len > 0) std::snprintf(dtype, (size_t)dtype_len, "%s", e.dtype.c_str());
  if (ndim) *ndim = (int)e.shape.size();
  for (int i = 0; shape && i < (int)e.shape.size() && i < max_dims; i++) shape[i] = e.shape[i];
  return MOERT_OK;
}

int moert_checkpoint_read_bf16(const moert_checkpoint* ck, const char* name, uint16_t* out, size_t n) {
  if (!ck || !name || !out) return set_error(MOERT_E_CONFIG, "checkpoint: null argument");
  std::vector<uint16_t> v;
  const int rc = read_bf16(ck, name, v, nullptr);
  if (rc) return rc;
  if (v.size() != n) return set_error(MOERT_E_CONFIG, "safetensors: %s holds %zu values, not %zu", name, v.size(), n);
  std::memcpy(out, v.data(), n * 2);
  return MOERT_OK;
}

int moert_checkpoint_load(const moert_checkpoint* ck, const moert_config* cfg, int wdtype, int embed_dtype,
                          moert_host_model** out) {
  if (!ck || !cfg || !out) return set_error(MOERT_E_CONFIG, "checkpoint: null argument");
  *out = nullptr;
  if (wdtype < MOERT_F32 || wdtype > MOERT_Q4_0 || embed_dtype < MOERT_F32 || embed_dtype > MOERT_Q4_0)
    return set_error(MOERT_E_CONFIG, "checkpoint: unknown dtype");
  const moert_config& c = *cfg;
  if (c.layers < 1 || c.hidden < 1 || c.heads < 1 || c.kv_heads < 1 || c.head_dim < 1 || c.experts < 1 ||
      c.inter < 1 || c.vocab < 1)
    return set_error(MOERT_E_CONFIG, "checkpoint: empty config");
  std::unique_ptr<moert_host_model> hm(new moert_host_model);
  hm->cfg = c;
  hm->wdtype = wdtype;
  hm->embed_dtype = embed_dtype;
  const uint64_t H = c.hidden, qd = (uint64_t)c.heads * c.head_dim, kvd = (uint64_t)c.kv_heads * c.head_dim,
                 I = c.inter, E = c.experts, V = c.vocab;
  // storage is reserved up front so that the pointers handed out stay valid
  hm->blobs.reserve((size_t)c.layers * 7 + 1);
  hm->f32s.reserve((size_t)c.layers * 2 + 1);
  hm->layers.resize(c.layers);
  auto mat = [&](const std::string& name, std::vector<uint64_t> shape, int dt, moert_tensor* t) -> int {
    hm->blobs.emplace_back();
    const int rc = read_matrix(ck, name, shape, dt, hm->blobs.back());
    if (rc) return rc;
    *t = moert_tensor{hm->blobs.back().data(), dt};
    return MOERT_OK;
  };
  auto vec = [&](const std::string& name, uint64_t n, const float** p) -> int {
    hm->f32s.emplace_back();
    const int rc = read_f32(ck, name, {n}, hm->f32s.back());
    if (rc) return rc;
    *p = hm->f32s.back().data();
    return MOERT_OK;
  };
  int rc;
  for (int l = 0; l < c.layers; l++) {
    const std::string p = "model.layers." + std::to_string(l);
    const std::string m = p + ".block_sparse_moe";
    moert_layer_weights& L = hm->layers[l];
    L.router_bias = nullptr;
    if ((rc = vec(p + ".input_layernorm.weight", H, &L.ln_attn)) ||
        (rc = vec(p + ".post_attention_layernorm.weight", H, &L.ln_moe)) ||
        (rc = mat(p + ".self_attn.q_proj.weight", {qd, H}, wdtype, &L.q)) ||
        (rc = mat(p + ".self_attn.k_proj.weight", {kvd, H}, wdtype, &L.k)) ||
        (rc = mat(p + ".self_attn.v_proj.weight", {kvd, H}, wdtype, &L.v)) ||
        (rc = mat(p + ".self_attn.o_proj.weight", {H, qd}, wdtype, &L.o)) ||
        (rc = mat(m + ".router.layer.weight", {E, H}, wdtype, &L.router)) ||
        (rc = mat(m + ".input_linear.weight", {E, 2 * I, H}, wdtype, &L.gate_up)) ||
        (rc = mat(m + ".output_linear.weight", {E, H, I}, wdtype, &L.down)))
      return rc;
  }
  const float* norm = nullptr;
  moert_tensor emb{};
  if ((rc = mat("model.embed_tokens.weight", {V, H}, embed_dtype, &emb)) || (rc = vec("model.norm.weight", H, &norm)))
    return rc;
  hm->w = moert_model_weights{emb, norm, hm->layers.data()};
  *out = hm.release();
  return MOERT_OK;
}

const moert_model_weights* moert_host_model_weights(const moert_host_model* hm) { return hm ? &hm->w : nullptr; }

int moert_host_model_config(const moert_host_model* hm, moert_config* cfg) {
  if (!hm || !cfg) return set_error(MOERT_E_CONFIG, "host model: null argument");
  *cfg = hm->cfg;
  return MOERT_OK;
}

int moert_host_model_destroy(moert_host_model* hm) {
  delete hm;
  return MOERT_OK;
}

}  // extern "C"
