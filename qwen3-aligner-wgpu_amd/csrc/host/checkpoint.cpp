// checkpoint.cpp -- see checkpoint.hpp.
#include "checkpoint.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>
#include <fstream>
#include <set>
#include <sstream>

#include "../half_bits.h"
#include "json_lite.hpp"
#include "qa.h"

namespace qah {

namespace {

thread_local std::string g_ckpt_err;

bool read_file(const std::string& path, std::string* out) {
  std::ifstream f(path, std::ios::binary);
  if (!f) return false;
  std::ostringstream ss;
  ss << f.rdbuf();
  *out = ss.str();
  return true;
}

bool file_exists(const std::string& path) {
  struct stat st;
  return ::stat(path.c_str(), &st) == 0 && S_ISREG(st.st_mode);
}

int elem_size(int dt) { return dt == ST_F32 ? 4 : (dt == ST_OTHER ? 0 : 2); }

// The 16-bit formats, round to nearest even.  f32 -> f16 by integer
// arithmetic (half_bits.h); f32 -> bf16 is the reference's
// (u + 0x7fff + ((u >> 16) & 1)) >> 16 (src/shaders.rs:169-179), with NaN
// kept a quiet NaN.
uint16_t to_f16(float v) { return qa_half::f16_from_f32(v); }
uint16_t to_bf16(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
float from_f16(uint16_t h) { return qa_half::f16_to_f32(h); }
float from_bf16(uint16_t h) { return __builtin_bit_cast(float, (uint32_t)h << 16); }

float load_elem(const uint8_t* p, int dt) {
  if (dt == ST_F32) {
    float v;
    std::memcpy(&v, p, 4);
    return v;
  }
  uint16_t h;
  std::memcpy(&h, p, 2);
  return dt == ST_F16 ? from_f16(h) : from_bf16(h);
}

// src/weights.rs:229-247: the `-hf` conversion's names onto the original ones.
std::string remap_hf(const std::string& n) {
  auto starts = [&](const char* p) { return n.rfind(p, 0) == 0; };
  auto rest = [&](const char* p) { return n.substr(std::strlen(p)); };
  if (starts("model.multi_modal_projector.linear_1"))
    return "thinker.audio_tower.proj1" + rest("model.multi_modal_projector.linear_1");
  if (starts("model.multi_modal_projector.linear_2"))
    return "thinker.audio_tower.proj2" + rest("model.multi_modal_projector.linear_2");
  if (starts("model.audio_tower.")) return "thinker.audio_tower." + rest("model.audio_tower.");
  if (starts("model.language_model.")) return "thinker.model." + rest("model.language_model.");
  if (starts("thinker.lm_head.")) return "score." + rest("thinker.lm_head.");
  return n;
}

}  // namespace

Checkpoint::~Checkpoint() {
  for (auto& m : maps_) ::munmap(m.first, m.second);
}

bool Checkpoint::map_shard(const std::string& path, std::string* err) {
  const int fd = ::open(path.c_str(), O_RDONLY);
  if (fd < 0) return *err = "cannot open " + path, false;
  struct stat st;
  if (::fstat(fd, &st) != 0 || st.st_size < 8) {
    ::close(fd);
    return *err = path + ": not a safetensors file (shorter than 8 bytes)", false;
  }
  const size_t size = (size_t)st.st_size;
  void* base = ::mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (base == MAP_FAILED) return *err = "cannot map " + path, false;
  maps_.emplace_back(base, size);
  const uint8_t* b = static_cast<const uint8_t*>(base);
  uint64_t hlen = 0;
  for (int i = 7; i >= 0; --i) hlen = (hlen << 8) | b[i];  // little-endian u64
  if (hlen > size - 8) return *err = path + ": header length past the end of the file", false;
  json::Value hdr;
  json::Parser ps(reinterpret_cast<const char*>(b + 8), (size_t)hlen);
  if (!ps.parse(&hdr) || hdr.kind != json::Value::Object)
    return *err = path + ": bad header JSON (" + ps.error() + ")", false;
  const uint8_t* data = b + 8 + hlen;
  const uint64_t dlen = size - 8 - hlen;
  for (const auto& f : hdr.fields) {
    if (f.first == "__metadata__") continue;
    const json::Value& t = f.second;
    const json::Value* dt = t.get("dtype");
    const json::Value* sh = t.get("shape");
    const json::Value* off = t.get("data_offsets");
    if (!dt || dt->kind != json::Value::String || !sh || sh->kind != json::Value::Array || !off ||
        off->kind != json::Value::Array || off->items.size() != 2 || !off->items[0].is_int() ||
        !off->items[1].is_int())
      return *err = path + ": bad header entry for " + f.first, false;
    StTensor st_;
    st_.dtype_name = dt->text;
    st_.dtype = dt->text == "F16" ? ST_F16 : dt->text == "BF16" ? ST_BF16
                : dt->text == "F32" ? ST_F32 : ST_OTHER;
    int64_t elems = 1;
    for (const auto& d : sh->items) {
      const int64_t n = d.is_int() ? d.as_int() : -1;
      // a dimension past 2^40, or a product past 2^48 elements, is no tensor of a model this size
      if (n < 0 || n > ((int64_t)1 << 40) || (n && elems > ((int64_t)1 << 48) / n))
        return *err = path + ": bad shape of " + f.first, false;
      elems *= n;
      st_.shape.push_back(n);
    }
    const uint64_t o0 = off->items[0].as_uint(), o1 = off->items[1].as_uint();
    if (o0 > o1 || o1 > dlen) return *err = path + ": data of " + f.first + " out of range", false;
    st_.data = data + o0;
    st_.bytes = (size_t)(o1 - o0);
    if (st_.dtype != ST_OTHER && (int64_t)st_.bytes != st_.numel() * elem_size(st_.dtype))
      return *err = path + ": " + f.first + " has " + std::to_string(st_.bytes) +
                    " bytes for its shape", false;
    if (!tensors_.emplace(f.first, std::move(st_)).second)
      return *err = "tensor " + f.first + " appears twice", false;
  }
  return true;
}

std::unique_ptr<Checkpoint> Checkpoint::open(const std::string& dir, std::string* err) {
  std::unique_ptr<Checkpoint> ck(new Checkpoint());
  const std::string index = dir + "/model.safetensors.index.json";
  if (file_exists(index)) {
    std::string text;
    json::Value idx;
    if (!read_file(index, &text)) return *err = "cannot read " + index, nullptr;
    json::Parser ps(text.data(), text.size());
    if (!ps.parse(&idx)) return *err = index + ": bad JSON (" + ps.error() + ")", nullptr;
    const json::Value* wm = idx.get("weight_map");
    if (!wm || wm->kind != json::Value::Object) return *err = index + ": no weight_map", nullptr;
    std::set<std::string> shards;  // sorted and deduplicated, as the reference does
    for (const auto& f : wm->fields)
      if (f.second.kind == json::Value::String) shards.insert(f.second.text);
    for (const auto& sh : shards)
      if (!ck->map_shard(dir + "/" + sh, err)) return nullptr;
  } else if (!ck->map_shard(dir + "/model.safetensors", err)) {
    return nullptr;
  }
  // src/weights.rs:249-264: remap only a checkpoint that uses `-hf` names
  bool hf = false;
  for (const auto& t : ck->tensors_) {
    const std::string& k = t.first;
    if (k.rfind("model.audio_tower.", 0) == 0 || k.rfind("model.language_model.", 0) == 0 ||
        k.rfind("thinker.lm_head.", 0) == 0)
      hf = true;
  }
  if (hf) {
    std::unordered_map<std::string, StTensor> m;
    for (auto& t : ck->tensors_) {
      const std::string k = remap_hf(t.first);
      if (!m.emplace(k, std::move(t.second)).second)
        return *err = "two tensors map to " + k, nullptr;
    }
    ck->tensors_.swap(m);
  }
  if (!read_file(dir + "/config.json", &ck->config_text_)) ck->config_text_.clear();
  return ck;
}

const StTensor* Checkpoint::find(const std::string& name) const {
  const auto it = tensors_.find(name);
  return it == tensors_.end() ? nullptr : &it->second;
}

bool Checkpoint::read_h16(const std::string& name, int dtype, uint16_t* dst, int64_t elems,
                          std::string* err) const {
  const StTensor* t = find(name);
  if (!t) return *err = "weight not found: " + name, false;
  if (dtype != QA_F16 && dtype != QA_BF16) return *err = "dtype must be QA_F16 or QA_BF16", false;
  if (t->dtype == ST_OTHER) return *err = name + ": unsupported dtype " + t->dtype_name, false;
  if (t->numel() != elems)
    return *err = name + ": " + std::to_string(t->numel()) + " elements, expected " +
                  std::to_string(elems), false;
  const int es = elem_size(t->dtype);
  if ((dtype == QA_F16 && t->dtype == ST_F16) || (dtype == QA_BF16 && t->dtype == ST_BF16)) {
    std::memcpy(dst, t->data, (size_t)elems * 2);  // safetensors is little-endian
    return true;
  }
  for (int64_t i = 0; i < elems; ++i) {
    const float v = load_elem(t->data + i * es, t->dtype);
    dst[i] = dtype == QA_F16 ? to_f16(v) : to_bf16(v);
  }
  return true;
}

bool Checkpoint::read_f32(const std::string& name, float* dst, int64_t elems,
                          std::string* err) const {
  const StTensor* t = find(name);
  if (!t) return *err = "weight not found: " + name, false;
  if (t->dtype == ST_OTHER) return *err = name + ": unsupported dtype " + t->dtype_name, false;
  if (t->numel() != elems)
    return *err = name + ": " + std::to_string(t->numel()) + " elements, expected " +
                  std::to_string(elems), false;
  const int es = elem_size(t->dtype);
  for (int64_t i = 0; i < elems; ++i) dst[i] = load_elem(t->data + i * es, t->dtype);
  return true;
}

bool Checkpoint::config(qah_ckpt_config* c, std::string* err) const {
  if (config_text_.empty()) return *err = "config.json missing or empty", false;
  json::Value root;
  json::Parser ps(config_text_.data(), config_text_.size());
  if (!ps.parse(&root) || root.kind != json::Value::Object)
    return *err = "config.json: bad JSON (" + ps.error() + ")", false;
  const json::Value* thinker = root.get("thinker_config");
  const json::Value* audio = thinker ? thinker->get("audio_config") : root.get("audio_config");
  const json::Value* text = thinker ? thinker->get("text_config") : root.get("text_config");
  if (!audio || !text)
    return *err = "config.json: neither thinker_config nor audio_config + text_config", false;
  const json::Value* ids = thinker ? thinker : &root;
  auto num = [](const json::Value* o, const char* k, double dflt) {
    const json::Value* v = o ? o->get(k) : nullptr;
    return v && v->kind == json::Value::Number ? v->as_double() : dflt;
  };
  auto inum = [&](const json::Value* o, const char* k, int64_t dflt) {
    const json::Value* v = o ? o->get(k) : nullptr;
    return v && v->kind == json::Value::Number ? v->as_int() : dflt;
  };
  // src/config.rs:36-150: field names and defaults
  c->vocab = inum(text, "vocab_size", 151936);
  c->hidden = inum(text, "hidden_size", 1024);
  c->inter = inum(text, "intermediate_size", 3072);
  c->layers = inum(text, "num_hidden_layers", 28);
  c->nqh = inum(text, "num_attention_heads", 16);
  c->nkvh = inum(text, "num_key_value_heads", 8);
  c->hd = inum(text, "head_dim", 128);
  c->rms_eps = num(text, "rms_norm_eps", 1e-6);
  c->rope_theta = num(text, "rope_theta", 1e6);
  if (const json::Value* rp = text->get("rope_parameters"))
    c->rope_theta = num(rp, "rope_theta", c->rope_theta);
  c->d_model = inum(audio, "d_model", 896);
  c->enc_layers = inum(audio, "encoder_layers", 18);
  c->enc_heads = inum(audio, "encoder_attention_heads", 14);
  c->enc_ffn = inum(audio, "encoder_ffn_dim", 3584);
  c->n_mels = inum(audio, "num_mel_bins", 128);
  c->c_conv = inum(audio, "downsample_hidden_size", 480);
  c->n_window = inum(audio, "n_window", 50);
  c->n_window_infer = inum(audio, "n_window_infer", 800);
  c->out_dim = inum(audio, "output_dim", 1024);
  c->audio_start = inum(ids, "audio_start_token_id", 151669);
  c->audio_end = inum(ids, "audio_end_token_id", 151670);
  c->audio_token = inum(ids, "audio_token_id", 151676);
  // src/config.rs:218-231: the head width is id2label's length (-hf) or
  // thinker_config.classify_num (original layout)
  const json::Value* i2l = root.get("id2label");
  if (i2l && i2l->kind == json::Value::Object)
    c->num_labels = (int64_t)i2l->fields.size();
  else
    c->num_labels = inum(thinker, "classify_num", 0);
  c->timestamp_token_id = inum(&root, "timestamp_token_id", -1);
  c->segment_ms = num(&root, "timestamp_segment_time", 80.0);
  return true;
}

namespace {

int feo(int frames) {
  auto d = [](int v) { return (v - 1) / 2 + 1; };
  return d(d(d(frames)));
}

struct Loader {
  const Checkpoint& ck;
  int dtype;
  std::string* err;
  int rc = QA_OK;

  bool h16(const std::string& name, std::vector<uint16_t>* v, int64_t n) {
    v->assign((size_t)n, 0);
    if (!ck.read_h16(name, dtype, v->data(), n, err)) return rc = QA_EINVAL, false;
    return true;
  }
  // a bias that may be absent (src/audio_encoder_gpu.rs:258-260): zeros then
  bool bias(const std::string& name, std::vector<uint16_t>* v, int64_t n) {
    if (!ck.find(name)) return v->assign((size_t)n, 0), true;
    return h16(name, v, n);
  }
  // a norm weight in the run's 16-bit format, widened for the f32 uploads
  bool h16f(const std::string& name, std::vector<float>* v, int64_t n) {
    std::vector<uint16_t> h;
    if (!h16(name, &h, n)) return false;
    v->resize((size_t)n);
    for (int64_t i = 0; i < n; ++i) (*v)[i] = dtype == QA_F16 ? from_f16(h[i]) : from_bf16(h[i]);
    return true;
  }
  bool f32(const std::string& name, std::vector<float>* v, int64_t n) {
    v->assign((size_t)n, 0.f);
    if (!ck.read_f32(name, v->data(), n, err)) return rc = QA_EINVAL, false;
    return true;
  }
  bool shape(const std::string& name, std::initializer_list<int64_t> want) {
    const StTensor* t = ck.find(name);
    if (!t) return *err = "weight not found: " + name, rc = QA_EINVAL, false;
    if (t->shape != std::vector<int64_t>(want)) {
      std::string s = name + ": shape [";
      for (size_t i = 0; i < t->shape.size(); ++i) s += (i ? ", " : "") + std::to_string(t->shape[i]);
      s += "], expected [";
      size_t i = 0;
      for (int64_t w : want) s += (i++ ? ", " : "") + std::to_string(w);
      *err = s + "]";
      return rc = QA_EINVAL, false;
    }
    return true;
  }
  bool call(int r, const char* what) {
    if (r == QA_OK) return true;
    *err = std::string(what) + " failed (" + std::to_string(r) + ")";
    return rc = r, false;
  }
};

}  // namespace

int tower_geometry(const qah_ckpt_config& c, double max_seconds, Geometry* g, std::string* err) {
  if (!(max_seconds > 0)) return *err = "max_seconds must be > 0", QA_EINVAL;
  // geometry the tower's kernels and the window formula need (a zero or
  // negative n_window would divide by zero below)
  if (c.n_window <= 0 || c.n_mels <= 0 || c.n_window_infer <= 0)
    return *err = "n_window, n_mels and n_window_infer must be positive", QA_EINVAL;
  if (c.n_window_infer < 2 * c.n_window)
    return *err = "n_window_infer is shorter than one chunk (2 n_window frames)", QA_EINVAL;
  if (c.hd != 128) return *err = "decoder heads must be 128 wide", QA_EUNSUPPORTED;
  if (c.nqh <= 0 || c.nkvh <= 0 || c.nqh % c.nkvh)
    return *err = "num_attention_heads must be a positive multiple of num_key_value_heads", QA_EINVAL;
  if (c.nqh / c.nkvh > 2)
    return *err = "GQA ratio num_attention_heads / num_key_value_heads above 2", QA_EUNSUPPORTED;
  g->cs = 2 * c.n_window;  // frames per chunk (src/audio_encoder.rs:770)
  // window = tokens per chunk x whole chunks per inference window
  // (src/audio_encoder.rs:807-810, src/audio_encoder_gpu.rs:883,1103)
  g->wlen = feo((int)g->cs) * (c.n_window_infer / g->cs);
  g->fdim = feo((int)c.n_mels);
  const int64_t max_samples = (int64_t)(max_seconds * 16000.0);
  g->max_chunks = (max_samples / 160 + g->cs - 1) / g->cs;
  return QA_OK;
}

int load_aligner(const Checkpoint& ck, qa_ctx* ctx, int dtype, double max_seconds, int max_rows,
                 qah_aenc** enc_out, qah_tdec** dec_out, qah_aligner** al_out, std::string* err) {
  qah_ckpt_config c{};
  if (!ck.config(&c, err)) return QA_EINVAL;
  if (dtype != QA_F16 && dtype != QA_BF16) return *err = "dtype must be QA_F16 or QA_BF16", QA_EINVAL;
  if (max_seconds <= 0 || max_rows <= 0) return *err = "max_seconds and max_rows must be > 0", QA_EINVAL;
  Geometry geo{};
  if (int rc = tower_geometry(c, max_seconds, &geo, err)) return rc;
  // what this build's kernels and the aligner's fixed token ids cover
  if (c.d_model != c.enc_heads * 64)
    return *err = "audio tower heads must be 64 wide", QA_EUNSUPPORTED;
  if (c.out_dim != c.hidden) return *err = "audio output_dim must equal hidden_size", QA_EINVAL;
  if (c.audio_start != 151669 || c.audio_end != 151670 || c.audio_token != 151676 ||
      c.timestamp_token_id != 151705)
    return *err = "token ids differ from the aligner's (151669 / 151670 / 151676 / 151705)",
           QA_EUNSUPPORTED;
  if (c.num_labels <= 0) return *err = "config.json gives no head width (id2label / classify_num)", QA_EINVAL;
  Loader L{ck, dtype, err};
  const std::string A = "thinker.audio_tower", T = "thinker.model";
  const int cs = (int)geo.cs, wlen = (int)geo.wlen, fdim = (int)geo.fdim;
  const int64_t max_samples = (int64_t)(max_seconds * 16000.0);
  const int max_chunks = (int)geo.max_chunks;
  const int64_t dm = c.d_model, cc = c.c_conv, ff = c.enc_ffn, hs = c.hidden, hd = c.hd;

  qah_aenc* enc = nullptr;
  qah_tdec* dec = nullptr;
  qah_aligner* al = nullptr;
  auto cleanup = [&](int code) {
    if (al) qah_aligner_destroy(al);
    if (enc) qah_aenc_destroy(enc);
    if (dec) qah_tdec_destroy(dec);
    return code;
  };
  if (!L.call(qah_aenc_create(ctx, dtype, (int)c.enc_layers, (int)c.n_mels, cs, (int)cc, (int)dm,
                              (int)c.enc_heads, (int)ff, (int)c.out_dim, wlen, max_chunks, &enc),
              "qah_aenc_create"))
    return cleanup(L.rc);
  std::vector<uint16_t> w, b, w2, b2, w3, b3;
  std::vector<float> f1, f2, f3, f4;
  // conv stem (src/audio_encoder_gpu.rs:743-746): [c_out][c_in][3][3] + bias
  for (int lv = 0; lv < 3; ++lv) {
    const std::string p = A + ".conv2d" + std::to_string(lv + 1);
    const int64_t cin = lv == 0 ? 1 : cc;
    if (!L.shape(p + ".weight", {cc, cin, 3, 3}) || !L.h16(p + ".weight", &w, cc * cin * 9) ||
        !L.shape(p + ".bias", {cc}) || !L.h16(p + ".bias", &b, cc) ||
        !L.call(qah_aenc_load_conv(enc, lv, w.data(), b.data()), "qah_aenc_load_conv"))
      return cleanup(L.rc);
  }
  if (!L.shape(A + ".conv_out.weight", {dm, cc * fdim}) ||
      !L.h16(A + ".conv_out.weight", &w, dm * cc * fdim) || !L.bias(A + ".conv_out.bias", &b, dm) ||
      !L.call(qah_aenc_load_conv_out(enc, w.data(), b.data()), "qah_aenc_load_conv_out"))
    return cleanup(L.rc);
  for (int li = 0; li < (int)c.enc_layers; ++li) {
    const std::string p = A + ".layers." + std::to_string(li);
    std::vector<uint16_t> qkv((size_t)(3 * dm * dm)), qkvb((size_t)(3 * dm));
    const char* parts[3] = {"q_proj", "k_proj", "v_proj"};  // fused q|k|v rows
    for (int j = 0; j < 3; ++j) {
      const std::string q = p + ".self_attn." + parts[j];
      if (!L.shape(q + ".weight", {dm, dm}) || !L.h16(q + ".weight", &w, dm * dm) ||
          !L.bias(q + ".bias", &b, dm))
        return cleanup(L.rc);
      std::copy(w.begin(), w.end(), qkv.begin() + j * dm * dm);
      std::copy(b.begin(), b.end(), qkvb.begin() + j * dm);
    }
    if (!L.h16f(p + ".self_attn_layer_norm.weight", &f1, dm) ||
        !L.h16f(p + ".self_attn_layer_norm.bias", &f2, dm) ||
        !L.h16f(p + ".final_layer_norm.weight", &f3, dm) ||
        !L.h16f(p + ".final_layer_norm.bias", &f4, dm) ||
        !L.shape(p + ".self_attn.out_proj.weight", {dm, dm}) ||
        !L.h16(p + ".self_attn.out_proj.weight", &w, dm * dm) ||
        !L.bias(p + ".self_attn.out_proj.bias", &b, dm) || !L.shape(p + ".fc1.weight", {ff, dm}) ||
        !L.h16(p + ".fc1.weight", &w2, ff * dm) || !L.bias(p + ".fc1.bias", &b2, ff) ||
        !L.shape(p + ".fc2.weight", {dm, ff}) || !L.h16(p + ".fc2.weight", &w3, dm * ff) ||
        !L.bias(p + ".fc2.bias", &b3, dm) ||
        !L.call(qah_aenc_load_layer(enc, li, f1.data(), f2.data(), qkv.data(), qkvb.data(), w.data(),
                                    b.data(), f3.data(), f4.data(), w2.data(), b2.data(),
                                    w3.data(), b3.data()),
                "qah_aenc_load_layer"))
      return cleanup(L.rc);
  }
  if (!L.h16f(A + ".ln_post.weight", &f1, dm) || !L.h16f(A + ".ln_post.bias", &f2, dm) ||
      !L.shape(A + ".proj1.weight", {dm, dm}) || !L.h16(A + ".proj1.weight", &w, dm * dm) ||
      !L.bias(A + ".proj1.bias", &b, dm) || !L.shape(A + ".proj2.weight", {c.out_dim, dm}) ||
      !L.h16(A + ".proj2.weight", &w2, c.out_dim * dm) || !L.bias(A + ".proj2.bias", &b2, c.out_dim) ||
      !L.call(qah_aenc_load_post(enc, f1.data(), f2.data(), w.data(), b.data(), w2.data(), b2.data()),
              "qah_aenc_load_post"))
    return cleanup(L.rc);

  // text decoder (src/decoder.rs:816-826): separate q / k / v and gate / up,
  // fused by the loader below it
  if (!L.call(qah_tdec_create(ctx, dtype, (int)c.layers, (int)hs, (int)c.nqh, (int)c.nkvh, (int)hd,
                              (int)c.inter, max_rows, (float)c.rms_eps, &dec),
              "qah_tdec_create"))
    return cleanup(L.rc);
  const int64_t qd = c.nqh * hd, kd = c.nkvh * hd, it = c.inter;
  std::vector<uint16_t> wq, wk, wv, wo, wg, wu, wd;
  for (int li = 0; li < (int)c.layers; ++li) {
    const std::string p = T + ".layers." + std::to_string(li);
    if (!L.shape(p + ".self_attn.q_proj.weight", {qd, hs}) ||
        !L.h16(p + ".self_attn.q_proj.weight", &wq, qd * hs) ||
        !L.shape(p + ".self_attn.k_proj.weight", {kd, hs}) ||
        !L.h16(p + ".self_attn.k_proj.weight", &wk, kd * hs) ||
        !L.shape(p + ".self_attn.v_proj.weight", {kd, hs}) ||
        !L.h16(p + ".self_attn.v_proj.weight", &wv, kd * hs) ||
        !L.shape(p + ".self_attn.o_proj.weight", {hs, qd}) ||
        !L.h16(p + ".self_attn.o_proj.weight", &wo, hs * qd) ||
        !L.shape(p + ".mlp.gate_proj.weight", {it, hs}) ||
        !L.h16(p + ".mlp.gate_proj.weight", &wg, it * hs) ||
        !L.shape(p + ".mlp.up_proj.weight", {it, hs}) ||
        !L.h16(p + ".mlp.up_proj.weight", &wu, it * hs) ||
        !L.shape(p + ".mlp.down_proj.weight", {hs, it}) ||
        !L.h16(p + ".mlp.down_proj.weight", &wd, hs * it) ||
        !L.h16f(p + ".input_layernorm.weight", &f1, hs) ||
        !L.h16f(p + ".post_attention_layernorm.weight", &f2, hs) ||
        !L.h16f(p + ".self_attn.q_norm.weight", &f3, hd) ||
        !L.h16f(p + ".self_attn.k_norm.weight", &f4, hd) ||
        !L.call(qah_tdec_load_layer(dec, li, wq.data(), wk.data(), wv.data(), wo.data(), wg.data(),
                                    wu.data(), wd.data(), f1.data(), f2.data(), f3.data(),
                                    f4.data()),
                "qah_tdec_load_layer"))
      return cleanup(L.rc);
  }
  {
    std::vector<float> cosv((size_t)max_rows * hd), sinv((size_t)max_rows * hd);
    // theta 1e6 whatever config.json says: the aligner builds its tables with
    // the constant (src/align_inference.rs:322-327); rope_theta only reaches
    // the reference's other forwards.  Rounded to the run's format (:371-372).
    if (!L.call(qa_rope_tables(max_rows, (int)hd, 1e6, (uint32_t)dtype, cosv.data(), sinv.data()),
                "qa_rope_tables") ||
        !L.call(qah_tdec_set_rope(dec, cosv.data(), sinv.data(), max_rows), "qah_tdec_set_rope"))
      return cleanup(L.rc);
  }
  // head (src/align_inference.rs:405-430): embedding in the run's format,
  // final norm and score in f32
  if (!L.call(qah_aligner_create(ctx, enc, dec, c.vocab, c.num_labels, c.segment_ms, max_samples, &al),
              "qah_aligner_create"))
    return cleanup(L.rc);
  if (!L.shape(T + ".embed_tokens.weight", {c.vocab, hs}) ||
      !L.h16(T + ".embed_tokens.weight", &w, c.vocab * hs) ||
      !L.call(qah_aligner_load_embed(al, w.data()), "qah_aligner_load_embed") ||
      !L.f32(T + ".norm.weight", &f1, hs) || !L.shape("score.weight", {c.num_labels, hs}) ||
      !L.f32("score.weight", &f2, c.num_labels * hs) ||
      !L.call(qah_aligner_load_head(al, f1.data(), f2.data()), "qah_aligner_load_head"))
    return cleanup(L.rc);
  *enc_out = enc;
  *dec_out = dec;
  *al_out = al;
  return QA_OK;
}

}  // namespace qah

extern "C" {

struct qah_ckpt {
  std::unique_ptr<qah::Checkpoint> c;
};

const char* qah_ckpt_error(void) { return qah::g_ckpt_err.c_str(); }

int qah_ckpt_open(const char* dir, qah_ckpt** out) {
  if (!dir || !out) return qah::g_ckpt_err = "qah_ckpt_open: null argument", QA_EINVAL;
  std::string err;
  auto ck = qah::Checkpoint::open(dir, &err);
  if (!ck) return qah::g_ckpt_err = err, QA_EINVAL;
  *out = new qah_ckpt{std::move(ck)};
  return QA_OK;
}

int qah_ckpt_tensor(qah_ckpt* c, const char* name, int* dtype, int* ndim, int64_t* shape) {
  if (!c || !name) return qah::g_ckpt_err = "qah_ckpt_tensor: null argument", QA_EINVAL;
  const qah::StTensor* t = c->c->find(name);
  if (!t) return qah::g_ckpt_err = std::string("weight not found: ") + name, QA_EINVAL;
  if (t->shape.size() > 8) return qah::g_ckpt_err = std::string(name) + ": more than 8 dims", QA_EUNSUPPORTED;
  if (dtype) *dtype = t->dtype;
  if (ndim) *ndim = (int)t->shape.size();
  if (shape)
    for (size_t i = 0; i < t->shape.size(); ++i) shape[i] = t->shape[i];
  return QA_OK;
}

int qah_ckpt_read_h16(qah_ckpt* c, const char* name, int dtype, uint16_t* dst, int64_t elems) {
  if (!c || !name || (!dst && elems)) return qah::g_ckpt_err = "qah_ckpt_read_h16: null argument", QA_EINVAL;
  std::string err;
  if (!c->c->read_h16(name, dtype, dst, elems, &err)) return qah::g_ckpt_err = err, QA_EINVAL;
  return QA_OK;
}

int qah_ckpt_read_f32(qah_ckpt* c, const char* name, float* dst, int64_t elems) {
  if (!c || !name || (!dst && elems)) return qah::g_ckpt_err = "qah_ckpt_read_f32: null argument", QA_EINVAL;
  std::string err;
  if (!c->c->read_f32(name, dst, elems, &err)) return qah::g_ckpt_err = err, QA_EINVAL;
  return QA_OK;
}

int qah_ckpt_read_config(qah_ckpt* c, qah_ckpt_config* out) {
  if (!c || !out) return qah::g_ckpt_err = "qah_ckpt_read_config: null argument", QA_EINVAL;
  std::string err;
  if (!c->c->config(out, &err)) return qah::g_ckpt_err = err, QA_EINVAL;
  return QA_OK;
}

int qah_ckpt_load_aligner(qah_ckpt* c, qa_ctx* ctx, int dtype, double max_seconds, int max_rows,
                          qah_aenc** enc, qah_tdec** dec, qah_aligner** al) {
  if (!c || !ctx || !enc || !dec || !al)
    return qah::g_ckpt_err = "qah_ckpt_load_aligner: null argument", QA_EINVAL;
  std::string err;
  const int rc = qah::load_aligner(*c->c, ctx, dtype, max_seconds, max_rows, enc, dec, al, &err);
  if (rc != QA_OK) qah::g_ckpt_err = err;
  return rc;
}

int qah_ckpt_geometry(qah_ckpt* c, double max_seconds, int64_t* out) {
  if (!c || !out) return qah::g_ckpt_err = "qah_ckpt_geometry: null argument", QA_EINVAL;
  std::string err;
  qah_ckpt_config cfg{};
  if (!c->c->config(&cfg, &err)) return qah::g_ckpt_err = err, QA_EINVAL;
  qah::Geometry g{};
  if (int rc = qah::tower_geometry(cfg, max_seconds, &g, &err)) return qah::g_ckpt_err = err, rc;
  out[0] = g.cs;
  out[1] = g.wlen;
  out[2] = g.fdim;
  out[3] = g.max_chunks;
  return QA_OK;
}

void qah_ckpt_close(qah_ckpt* c) { delete c; }

}  // extern "C"
