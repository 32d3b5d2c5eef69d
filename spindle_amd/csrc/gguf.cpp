// GGUF v2/v3 files (the llama.cpp model format) for the engine: the reader of
// GgufModelIndex::parse_file (gguf_loader.rs:142-247) over a read-only mapping of the file, the
// hyperparameters of ModelConfig::from_gguf (smollm_chat.rs:69-120), and the engine load of
// load_with_index_sharded (:1905-2154) with resolve_layers' tensor names (:214-284): every
// tensor is uploaded straight from the mapping (the GGUF block bytes the reference borrows
// from its mmap). Host code only; the upload is spx_engine_set_tensor's.
#include <fcntl.h>
#include <stdint.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdio>

#include <algorithm>
#include <map>
#include <new>
#include <string>
#include <vector>

#include "../../include/spx.h"
#include "internal.h"

namespace {

enum : uint32_t { GV_U8, GV_I8, GV_U16, GV_I16, GV_U32, GV_I32, GV_F32, GV_BOOL, GV_STR, GV_ARR, GV_U64, GV_I64, GV_F64 };

struct Value {
  uint32_t type = 0;
  uint64_t u = 0;   // unsigned integers and bool
  int64_t i = 0;    // signed integers
  double f = 0.0;   // f32 / f64
  std::string s;
  uint32_t elem = 0;        // arrays: element type and count
  uint64_t count = 0;
  std::vector<std::string> strs;  // kept for tokenizer.ggml.tokens only

  // GgufValue::as_usize (gguf_loader.rs:88-101): integers that are not negative
  bool as_index(uint64_t &out) const {
    switch (type) {
    case GV_U8: case GV_U16: case GV_U32: case GV_U64: out = u; return true;
    case GV_I8: case GV_I16: case GV_I32: case GV_I64: if (i < 0) return false; out = (uint64_t)i; return true;
    default: return false;
    }
  }
  // GgufValue::as_f32 (:104-110): floats, or an index as f32
  bool as_f32(float &out) const {
    if (type == GV_F32 || type == GV_F64) { out = (float)f; return true; }
    uint64_t v;
    if (!as_index(v)) return false;
    out = (float)v;
    return true;
  }
};

struct Tensor {
  std::string name;
  std::vector<uint64_t> dims;
  uint32_t dtype = 0;
  uint64_t rel = 0, abs = 0;
};

struct Reader {
  const uint8_t *p, *end;
  std::string err;
  bool need(uint64_t n) {
    if ((uint64_t)(end - p) < n) { if (err.empty()) err = "truncated GGUF header"; return false; }
    return true;
  }
  template <class T> bool get(T &v) {
    if (!need(sizeof(T))) return false;
    memcpy(&v, p, sizeof(T));
    p += sizeof(T);
    return true;
  }
  bool str(std::string &s, bool keep = true) {  // read_gguf_string (:394-405): u64 length, at most 16 MiB
    uint64_t n;
    if (!get(n)) return false;
    if (n > (16u << 20)) { err = "GGUF string length exceeds 16 MiB"; return false; }
    if (!need(n)) return false;
    if (keep) s.assign(reinterpret_cast<const char *>(p), (size_t)n);
    p += n;
    return true;
  }
};

int elem_size(uint32_t t) {  // skip_scalar_elem (:407-417)
  switch (t) {
  case GV_U8: case GV_I8: case GV_BOOL: return 1;
  case GV_U16: case GV_I16: return 2;
  case GV_U32: case GV_I32: case GV_F32: return 4;
  case GV_U64: case GV_I64: case GV_F64: return 8;
  default: return 0;
  }
}

bool read_value(Reader &r, const std::string &key, Value &v) {  // read_gguf_value (:419-479)
  if (!r.get(v.type)) return false;
  switch (v.type) {
  case GV_U8: { uint8_t x; if (!r.get(x)) return false; v.u = x; return true; }
  case GV_I8: { int8_t x; if (!r.get(x)) return false; v.i = x; return true; }
  case GV_U16: { uint16_t x; if (!r.get(x)) return false; v.u = x; return true; }
  case GV_I16: { int16_t x; if (!r.get(x)) return false; v.i = x; return true; }
  case GV_U32: { uint32_t x; if (!r.get(x)) return false; v.u = x; return true; }
  case GV_I32: { int32_t x; if (!r.get(x)) return false; v.i = x; return true; }
  case GV_F32: { float x; if (!r.get(x)) return false; v.f = x; return true; }
  case GV_BOOL: { uint8_t x; if (!r.get(x)) return false; v.u = x != 0; return true; }
  case GV_STR: return r.str(v.s);
  case GV_U64: return r.get(v.u);
  case GV_I64: return r.get(v.i);
  case GV_F64: return r.get(v.f);
  case GV_ARR: {
    if (!r.get(v.elem) || !r.get(v.count)) return false;
    if (v.elem == GV_STR) {
      const bool keep = key == "tokenizer.ggml.tokens";
      if (keep) v.strs.reserve((size_t)std::min<uint64_t>(v.count, 1u << 20));
      for (uint64_t k = 0; k < v.count; k++) {
        std::string s;
        if (!r.str(s, keep)) return false;
        if (keep) v.strs.push_back(std::move(s));
      }
      return true;
    }
    const int es = elem_size(v.elem);
    if (!es) { r.err = "unknown GGUF array elem"; return false; }
    if (v.count > (uint64_t)(r.end - r.p) / (uint64_t)es) { r.err = "truncated GGUF header"; return false; }
    r.p += v.count * es;
    return true;
  }
  default: r.err = "unknown GGUF value type " + std::to_string(v.type); return false;
  }
}

}  // namespace

struct spx_gguf {
  int fd = -1;
  const uint8_t *base = nullptr;
  size_t size = 0;
  uint32_t version = 0;
  uint64_t alignment = 32, data_off = 0;
  std::string arch, name;
  std::map<std::string, Value> meta;
  std::vector<std::string> vocab;
  std::vector<Tensor> tensors;
  std::map<std::string, int64_t> by_name;

  const Value *get(const std::string &k) const {
    auto it = meta.find(k);
    return it == meta.end() ? nullptr : &it->second;
  }
  const Tensor *find(const std::string &n) const {
    auto it = by_name.find(n);
    return it == by_name.end() ? nullptr : &tensors[it->second];
  }
  ~spx_gguf() {
    if (base) munmap(const_cast<uint8_t *>(base), size);
    if (fd >= 0) close(fd);
  }
};

namespace {

int parse(spx_gguf *g) {
  Reader r{g->base, g->base + g->size, {}};
  uint32_t magic;
  if (!r.get(magic)) return spx::fail("not a GGUF file (too short)");
  if (magic != 0x46554747u) {  // "GGUF"
    char b[64];
    snprintf(b, sizeof b, "not a GGUF file (magic = %#x)", magic);
    return spx::fail(b);
  }
  uint64_t n_tensors, n_kv;
  if (!r.get(g->version) || !r.get(n_tensors) || !r.get(n_kv)) return spx::fail(r.err);
  for (uint64_t k = 0; k < n_kv; k++) {
    std::string key;
    Value v;
    if (!r.str(key) || !read_value(r, key, v)) return spx::fail(r.err);
    if (key == "tokenizer.ggml.tokens" && v.type == GV_ARR && v.elem == GV_STR) g->vocab = v.strs;
    v.strs.clear();
    g->meta[key] = std::move(v);
  }
  if (const Value *a = g->get("general.alignment")) {  // (:186-190) U32 or U64, at least 32
    if (a->type == GV_U32 || a->type == GV_U64) {
      // a power of two of at most 1 GiB (ggml's rule): the padding below cannot wrap
      if (a->u == 0 || (a->u & (a->u - 1)) != 0 || a->u > (1ull << 30))
        return spx::fail("general.alignment " + std::to_string(a->u) + " is not a power of two of at most 1 GiB");
      g->alignment = std::max<uint64_t>(a->u, 32);
    }
  }
  const Value *ar = g->get("general.architecture");
  g->arch = ar && ar->type == GV_STR ? ar->s : "";
  const Value *nm = g->get("general.name");
  g->name = nm && nm->type == GV_STR ? nm->s : "";
  for (uint64_t k = 0; k < n_tensors; k++) {  // (:200-216)
    Tensor t;
    uint32_t nd;
    if (!r.str(t.name) || !r.get(nd)) return spx::fail(r.err);
    if (nd < 1 || nd > 4) return spx::fail("tensor " + t.name + ": " + std::to_string(nd) + " dimensions");
    t.dims.resize(nd);
    for (auto &d : t.dims)
      if (!r.get(d)) return spx::fail(r.err);
    if (!r.get(t.dtype) || !r.get(t.rel)) return spx::fail(r.err);
    g->by_name[t.name] = (int64_t)g->tensors.size();
    g->tensors.push_back(std::move(t));
  }
  const uint64_t header_end = (uint64_t)(r.p - g->base);
  g->data_off = (header_end + g->alignment - 1) / g->alignment * g->alignment;  // (:219-221)
  for (auto &t : g->tensors)
    if (__builtin_add_overflow(g->data_off, t.rel, &t.abs))
      return spx::fail("tensor " + t.name + ": data offset " + std::to_string(t.rel) + " overflows");
  return 0;
}

// rows = dims[1] * dims[2] * dims[3]; -1 when a dimension or the product leaves int64
int64_t tensor_rows(const Tensor &t) {
  int64_t n = 1;
  for (size_t k = 1; k < t.dims.size(); k++)
    if (t.dims[k] > (uint64_t)INT64_MAX || __builtin_mul_overflow(n, (int64_t)t.dims[k], &n)) return -1;
  return n;
}

}  // namespace

extern "C" {

int spx_gguf_open(const char *path, spx_gguf **out) {
  if (!path || !out) return spx::fail("spx_gguf_open: null argument");
  *out = nullptr;
  spx_gguf *g = new (std::nothrow) spx_gguf();
  if (!g) return spx::fail("spx_gguf_open: out of memory");
  g->fd = open(path, O_RDONLY);
  struct stat st;
  if (g->fd < 0 || fstat(g->fd, &st) != 0) {
    delete g;
    return spx::fail(std::string("spx_gguf_open: cannot open ") + path);
  }
  g->size = (size_t)st.st_size;
  if (g->size > 0) {
    void *m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (m == MAP_FAILED) {
      delete g;
      return spx::fail(std::string("spx_gguf_open: cannot map ") + path);
    }
    g->base = static_cast<const uint8_t *>(m);
  }
  if (int rc = parse(g)) {
    delete g;
    return rc;
  }
  *out = g;
  return 0;
}

int spx_gguf_close(spx_gguf *g) {
  delete g;
  return 0;
}

int spx_gguf_info(const spx_gguf *g, uint32_t *version, uint64_t *alignment, uint64_t *data_offset, int64_t *n_tensors,
                  int64_t *n_meta) {
  if (!g) return spx::fail("spx_gguf_info: null file");
  if (version) *version = g->version;
  if (alignment) *alignment = g->alignment;
  if (data_offset) *data_offset = g->data_off;
  if (n_tensors) *n_tensors = (int64_t)g->tensors.size();
  if (n_meta) *n_meta = (int64_t)g->meta.size();
  return 0;
}

int spx_gguf_tensor(const spx_gguf *g, int64_t i, const char **name, int *dtype, int *n_dims, uint64_t *dims,
                    uint64_t *abs_offset) {
  if (!g || i < 0 || i >= (int64_t)g->tensors.size()) return spx::fail("spx_gguf_tensor: no such tensor");
  const Tensor &t = g->tensors[i];
  if (name) *name = t.name.c_str();
  if (dtype) *dtype = (int)t.dtype;
  if (n_dims) *n_dims = (int)t.dims.size();
  if (dims)
    for (size_t k = 0; k < 4; k++) dims[k] = k < t.dims.size() ? t.dims[k] : 1;
  if (abs_offset) *abs_offset = t.abs;
  return 0;
}

int64_t spx_gguf_find(const spx_gguf *g, const char *name) {
  if (!g || !name) return -1;
  auto it = g->by_name.find(name);
  return it == g->by_name.end() ? -1 : it->second;
}

int spx_gguf_meta_type(const spx_gguf *g, const char *key) {
  const Value *v = g && key ? g->get(key) : nullptr;
  return v ? (int)v->type : -1;
}

int spx_gguf_meta_index(const spx_gguf *g, const char *key, uint64_t *out) {
  const Value *v = g && key ? g->get(key) : nullptr;
  if (!v || !out || !v->as_index(*out)) return spx::fail(std::string("spx_gguf_meta_index: no non-negative integer ") + (key ? key : ""));
  return 0;
}

int spx_gguf_meta_f32(const spx_gguf *g, const char *key, float *out) {
  const Value *v = g && key ? g->get(key) : nullptr;
  if (!v || !out || !v->as_f32(*out)) return spx::fail(std::string("spx_gguf_meta_f32: no number ") + (key ? key : ""));
  return 0;
}

int spx_gguf_meta_bool(const spx_gguf *g, const char *key, int *out) {
  const Value *v = g && key ? g->get(key) : nullptr;
  if (!v || !out || v->type != GV_BOOL) return spx::fail(std::string("spx_gguf_meta_bool: no bool ") + (key ? key : ""));
  *out = (int)v->u;
  return 0;
}

int spx_gguf_meta_str(const spx_gguf *g, const char *key, const char **out) {
  const Value *v = g && key ? g->get(key) : nullptr;
  if (!v || !out || v->type != GV_STR) return spx::fail(std::string("spx_gguf_meta_str: no string ") + (key ? key : ""));
  *out = v->s.c_str();
  return 0;
}

int spx_gguf_meta_array(const spx_gguf *g, const char *key, int *elem_type, uint64_t *count) {
  const Value *v = g && key ? g->get(key) : nullptr;
  if (!v || v->type != GV_ARR) return spx::fail(std::string("spx_gguf_meta_array: no array ") + (key ? key : ""));
  if (elem_type) *elem_type = (int)v->elem;
  if (count) *count = v->count;
  return 0;
}

int64_t spx_gguf_vocab_size(const spx_gguf *g) { return g ? (int64_t)g->vocab.size() : -1; }

const char *spx_gguf_token(const spx_gguf *g, int64_t id) {
  return g && id >= 0 && id < (int64_t)g->vocab.size() ? g->vocab[(size_t)id].c_str() : nullptr;
}

int spx_gguf_config(const spx_gguf *g, spx_model_config *c) {
  if (!g || !c) return spx::fail("spx_gguf_config: null argument");
  const std::string &arch = g->arch;
  auto get = [&](const char *k) { return g->get(arch + "." + k); };
  auto num = [&](const char *k, uint64_t &v) { const Value *x = get(k); return x && x->as_index(v); };
  auto f32 = [&](const char *k, float dflt) { const Value *x = get(k); float v; return x && x->as_f32(v) ? v : dflt; };
  int neox;
  if (arch == "llama" || arch == "granite" || arch == "granitemoe") neox = 0;
  else if (arch == "qwen2" || arch == "qwen2moe" || arch == "qwen3" || arch == "qwen3moe" || arch == "olmoe") neox = 1;
  else return spx::fail("unsupported architecture `" + arch + "`");
  uint64_t gating;
  if (num("expert_gating_func", gating) && gating != 1) return spx::fail("only softmax expert gating is supported");
  uint64_t dim, n_heads, n_layers;
  if (!num("embedding_length", dim)) return spx::fail("GGUF metadata missing `" + arch + ".embedding_length`");
  if (!num("attention.head_count", n_heads)) return spx::fail("GGUF metadata missing `" + arch + ".attention.head_count`");
  if (!num("block_count", n_layers)) return spx::fail("GGUF metadata missing `" + arch + ".block_count`");
  if (n_heads == 0) return spx::fail("attention.head_count is 0");
  uint64_t n_kv = n_heads, hd = dim / n_heads, n_exp = 0, n_used = 0, ctx = 2048;
  num("attention.head_count_kv", n_kv);
  num("attention.key_length", hd);
  num("expert_count", n_exp);
  num("expert_used_count", n_used);
  num("context_length", ctx);
  memset(c, 0, sizeof *c);
  c->dim = (int)dim;
  c->n_heads = (int)n_heads;
  c->n_kv_heads = (int)n_kv;
  c->head_dim = (int)hd;
  c->n_layers = (int)n_layers;
  int64_t vocab = (int64_t)g->vocab.size();
  if (vocab == 0) {  // no tokenizer table: the embedding's rows
    const Tensor *e = g->find("token_embd.weight");
    vocab = e && e->dims.size() >= 2 ? (int64_t)e->dims[1] : 0;
  }
  c->vocab = (int)vocab;
  c->max_seq = (int)std::min<uint64_t>(ctx, INT32_MAX);
  c->rope_theta = f32("rope.freq_base", 10000.0f);
  c->rms_eps = f32("attention.layer_norm_rms_epsilon", 1e-5f);
  c->rope_neox = neox;
  c->n_expert = (int)n_exp;
  c->n_expert_used = (int)std::min(n_used, n_exp);
  const Value *en = get("expert_weights_norm");  // Qwen2-MoE and OLMoE do not renormalise
  c->expert_norm = en && en->type == GV_BOOL ? (int)en->u : !(arch == "qwen2moe" || arch == "olmoe");
  c->moe_prune = 0.0f;
  c->embedding_scale = f32("embedding_scale", 1.0f);
  c->residual_scale = f32("residual_scale", 1.0f);
  c->logit_scale = f32("logit_scale", 1.0f);
  c->attn_scale = f32("attention.scale", 0.0f);  // 0: 1/sqrt(head_dim)
  if (hd % 8 != 0 || n_kv == 0 || n_heads % n_kv != 0) return spx::fail("unsupported head layout");
  return 0;
}

// (:1925-1936) eos, then the ids of <|endoftext|>, <|im_end|>, <|end_of_text|>, without repeats
int spx_gguf_stop_ids(const spx_gguf *g, int32_t *ids, int cap, int *n) {
  if (!g || !n || (cap > 0 && !ids)) return spx::fail("spx_gguf_stop_ids: null argument");
  std::vector<int64_t> out;
  auto add = [&](int64_t id) { if (id >= 0 && std::find(out.begin(), out.end(), id) == out.end()) out.push_back(id); };
  uint64_t eos;
  if (const Value *v = g->get("tokenizer.ggml.eos_token_id"))
    if (v->as_index(eos)) add((int64_t)eos);
  for (const char *s : {"<|endoftext|>", "<|im_end|>", "<|end_of_text|>"}) {
    auto it = std::find(g->vocab.begin(), g->vocab.end(), s);
    if (it != g->vocab.end()) add(it - g->vocab.begin());
  }
  *n = (int)out.size();
  for (int i = 0; i < std::min(cap, *n); i++) ids[i] = (int32_t)out[i];
  return 0;
}

// (:1937) the ids of <think> and </think> (-1 when the vocabulary has no such pair)
int spx_gguf_think_ids(const spx_gguf *g, int32_t *open_id, int32_t *close_id) {
  if (!g || !open_id || !close_id) return spx::fail("spx_gguf_think_ids: null argument");
  auto a = std::find(g->vocab.begin(), g->vocab.end(), "<think>"), b = std::find(g->vocab.begin(), g->vocab.end(), "</think>");
  const bool both = a != g->vocab.end() && b != g->vocab.end();
  *open_id = both ? (int32_t)(a - g->vocab.begin()) : -1;
  *close_id = both ? (int32_t)(b - g->vocab.begin()) : -1;
  return 0;
}

// (:1944-1963) every tensor's rows end within the file
int spx_gguf_check(const spx_gguf *g) {
  if (!g) return spx::fail("spx_gguf_check: null file");
  uint64_t needed = 0;
  for (const auto &t : g->tensors) {
    if (t.dims[0] > (uint64_t)INT64_MAX) return spx::fail("tensor " + t.name + ": dims[0] out of range");
    const int64_t rb = spx::row_bytes((int)t.dtype, (int64_t)t.dims[0]), rows = tensor_rows(t);
    if (rb <= 0) continue;
    uint64_t bytes = 0;
    if (rows < 0 || __builtin_mul_overflow((uint64_t)rb, (uint64_t)rows, &bytes) || t.abs > g->size || bytes > g->size - t.abs)
      return spx::fail("the file is incomplete: tensor " + t.name + " does not fit in its " + std::to_string(g->size >> 20) + " MiB");
    needed = std::max(needed, t.abs + bytes);
  }
  if (needed > g->size)
    return spx::fail("the file is incomplete: it is " + std::to_string(g->size >> 20) + " MiB but its tensors need " +
                     std::to_string(needed >> 20) + " MiB");
  return 0;
}

int spx_engine_load_gguf(spx_ctx *ctx, const spx_gguf *g, int max_seq, float moe_prune, spx_engine **out) {
  if (!ctx || !g || !out) return spx::fail("spx_engine_load_gguf: null argument");
  *out = nullptr;
  spx_model_config c;
  if (int r = spx_gguf_config(g, &c)) return r;
  if (int r = spx_gguf_check(g)) return r;
  if (max_seq > 0) c.max_seq = max_seq;
  c.moe_prune = moe_prune;
  // resolve_layers (:214-284): what this engine runs, and the layouts it refuses
  std::vector<std::string> names = {"token_embd.weight", "output_norm.weight"};
  if (g->find("output.weight")) names.push_back("output.weight");  // else tied (:1921)
  for (int l = 0; l < c.n_layers; l++) {
    const std::string p = "blk." + std::to_string(l) + ".";
    auto has = [&](const char *s) { return g->find(p + s) != nullptr; };
    for (const char *s : {"attn_norm.weight", "attn_q.weight", "attn_k.weight", "attn_v.weight", "attn_output.weight", "ffn_norm.weight"})
      names.push_back(p + s);
    for (const char *s : {"attn_q.bias", "attn_k.bias", "attn_v.bias", "attn_q_norm.weight", "attn_k_norm.weight"})
      if (has(s)) names.push_back(p + s);
    if (has("attn_q_norm.weight")) {
      const Tensor *qn = g->find(p + "attn_q_norm.weight");
      if ((int64_t)qn->dims[0] == (int64_t)c.n_heads * c.head_dim && c.n_heads * c.head_dim != c.head_dim)
        return spx::fail(p + "attn_q_norm.weight covers the whole projection (OLMoE); only per-head norms are supported");
    }
    if (has("ffn_gate_inp.weight")) {
      if (has("ffn_gate_shexp.weight")) return spx::fail(p + ": shared experts are not supported");
      if (c.n_expert == 0 || c.n_expert_used == 0) return spx::fail("MoE tensors present but expert_count/expert_used_count missing");
      for (const char *s : {"ffn_gate_inp.weight", "ffn_gate_exps.weight", "ffn_up_exps.weight", "ffn_down_exps.weight"}) names.push_back(p + s);
    } else if (has("ffn_gate.0.weight")) {
      return spx::fail("old per-expert Mixtral layout (ffn_gate.N) is not supported; re-convert the GGUF");
    } else {
      for (const char *s : {"ffn_gate.weight", "ffn_up.weight", "ffn_down.weight"}) names.push_back(p + s);
    }
  }
  spx_engine *e = nullptr;
  if (int r = spx_engine_create(ctx, &c, &e)) return r;
  for (const auto &n : names) {
    const Tensor *t = g->find(n);
    int r = 0;
    if (!t) r = spx::fail("missing tensor " + n);
    else {
      const int64_t cols = (int64_t)t->dims[0], rows = t->dims.size() > 1 ? (int64_t)t->dims[1] : 1;
      const int ne = t->dims.size() > 2 ? (int)t->dims[2] : 1;
      r = spx_engine_set_tensor(e, n.c_str(), (int)t->dtype, cols, rows, ne, g->base + t->abs);
    }
    if (r) {
      const std::string msg = spx_last_error();
      spx_engine_destroy(e);
      return spx::fail(msg);
    }
  }
  if (spx_engine_prepare(e) != 0) {
    const std::string msg = spx_last_error();
    spx_engine_destroy(e);
    return spx::fail(msg);
  }
  *out = e;
  return 0;
}

}  // extern "C"
