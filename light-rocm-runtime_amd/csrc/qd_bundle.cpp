// Weight-bundle I/O (see qd_bundle.hpp). The manifest is parsed with a small
// strict JSON reader; the validation rules and the diagnostics follow
// executor/qwen/weight_bundle.hpp:74-154,460-602 so callers see the same
// errors, and the writer emits the same text as weight_bundle.hpp:604-757.
#include "qd_bundle.hpp"

#include <cerrno>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <limits>
#include <map>
#include <memory>
#include <sstream>
#include <stdexcept>
#include <utility>

namespace qd::bundle {

const char *const kLayerTensorNames[kLayerTensorCount] = {
    "attention_norm_weight", "mlp_norm_weight", "q_weight",    "k_weight",
    "v_weight",              "q_bias",          "k_bias",      "v_bias",
    "out_weight",            "gate_weight",     "up_weight",   "down_weight"};

namespace {

// ---- minimal JSON -------------------------------------------------------------
struct Json {
  enum Kind { kNull, kBool, kNumber, kString, kArray, kObject } kind = kNull;
  std::string text;  // number literal or string value
  bool boolean = false;
  std::vector<Json> items;
  std::vector<std::pair<std::string, Json>> members;

  const Json *get(const std::string &key) const {
    for (const auto &m : members)
      if (m.first == key) return &m.second;
    return nullptr;
  }
};

class Parser {
 public:
  explicit Parser(const std::string &s) : s_(s) {}
  Json parse() {
    Json v = value();
    ws();
    if (i_ != s_.size()) fail("trailing characters");
    return v;
  }

 private:
  [[noreturn]] void fail(const char *what) {
    throw std::runtime_error(std::string("invalid weight manifest JSON: ") +
                             what + " at offset " + std::to_string(i_));
  }
  void ws() {
    while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\n' ||
                              s_[i_] == '\r' || s_[i_] == '\t'))
      ++i_;
  }
  bool eat(char c) {
    ws();
    if (i_ < s_.size() && s_[i_] == c) {
      ++i_;
      return true;
    }
    return false;
  }
  Json value() {
    ws();
    if (i_ >= s_.size()) fail("unexpected end");
    const char c = s_[i_];
    Json v;
    if (c == '{') {
      ++i_;
      v.kind = Json::kObject;
      if (eat('}')) return v;
      do {
        ws();
        std::string key = string();
        if (!eat(':')) fail("expected ':'");
        v.members.emplace_back(std::move(key), value());
      } while (eat(','));
      if (!eat('}')) fail("expected '}'");
    } else if (c == '[') {
      ++i_;
      v.kind = Json::kArray;
      if (eat(']')) return v;
      do {
        v.items.push_back(value());
      } while (eat(','));
      if (!eat(']')) fail("expected ']'");
    } else if (c == '"') {
      v.kind = Json::kString;
      v.text = string();
    } else if (s_.compare(i_, 4, "true") == 0) {
      i_ += 4;
      v.kind = Json::kBool;
      v.boolean = true;
    } else if (s_.compare(i_, 5, "false") == 0) {
      i_ += 5;
      v.kind = Json::kBool;
    } else if (s_.compare(i_, 4, "null") == 0) {
      i_ += 4;
    } else if (c == '-' || (c >= '0' && c <= '9')) {
      const size_t b = i_;
      while (i_ < s_.size() &&
             (std::strchr("+-.eE", s_[i_]) || (s_[i_] >= '0' && s_[i_] <= '9')))
        ++i_;
      v.kind = Json::kNumber;
      v.text = s_.substr(b, i_ - b);
    } else {
      fail("unexpected character");
    }
    return v;
  }
  std::string string() {
    if (i_ >= s_.size() || s_[i_] != '"') fail("expected string");
    ++i_;
    std::string out;
    while (i_ < s_.size() && s_[i_] != '"') {
      if (s_[i_] == '\\') {
        if (++i_ >= s_.size()) fail("bad escape");
        const char e = s_[i_];
        out += e == 'n' ? '\n' : e == 't' ? '\t' : e;
      } else {
        out += s_[i_];
      }
      ++i_;
    }
    if (i_ >= s_.size()) fail("unterminated string");
    ++i_;
    return out;
  }
  const std::string &s_;
  size_t i_ = 0;
};

// ---- helpers --------------------------------------------------------------------
std::vector<unsigned char> read_file(const std::string &path,
                                     const std::string &what) {
  std::ifstream f(path, std::ios::binary | std::ios::ate);
  if (!f) throw std::runtime_error("failed to open " + what + " file: " + path);
  const std::streamsize size = f.tellg();
  if (size <= 0) throw std::runtime_error(what + " file is empty: " + path);
  f.seekg(0, std::ios::beg);
  std::vector<unsigned char> data(static_cast<size_t>(size));
  if (!f.read(reinterpret_cast<char *>(data.data()), size))
    throw std::runtime_error("failed to read " + what + " file: " + path);
  return data;
}

size_t checked_mul(size_t a, size_t b, const std::string &ctx) {
  if (a != 0 && b > std::numeric_limits<size_t>::max() / a)
    throw std::overflow_error(ctx + " overflows size_t");
  return a * b;
}

// The data file must be a plain relative name under the manifest directory
// (weight_bundle.hpp:123-154).
std::string data_path(const std::string &manifest, const std::string &name,
                      const std::string &what) {
  bool parent = false;
  size_t b = 0;
  while (b <= name.size()) {
    const size_t e = name.find('/', b);
    if (name.substr(b, e == std::string::npos ? std::string::npos : e - b) == "..")
      parent = true;
    if (e == std::string::npos) break;
    b = e + 1;
  }
  if (name.empty() || name[0] == '/' || parent)
    throw std::runtime_error("invalid " + what + " data path: " + name);
  const size_t slash = manifest.find_last_of('/');
  return slash == std::string::npos ? name : manifest.substr(0, slash + 1) + name;
}

struct Doc {
  Json root;
  std::string what;  // "mini decoder weight" / "mini model tail"

  const Json &field(const char *name) const {
    const Json *v = root.get(name);
    if (!v) throw std::runtime_error("missing " + what + " manifest field: " + name);
    return *v;
  }
  std::string str(const char *name) const {
    const Json &v = field(name);
    if (v.kind != Json::kString)
      throw std::runtime_error(what + " manifest field is not a string: " + name);
    return v.text;
  }
};

uint64_t parse_uint(const Json &v, uint64_t limit, const std::string &err) {
  if (v.kind != Json::kNumber || v.text.empty()) throw std::runtime_error(err);
  uint64_t value = 0;
  for (char c : v.text) {
    if (c < '0' || c > '9') throw std::runtime_error(err);
    const uint64_t d = static_cast<uint64_t>(c - '0');
    if (value > (limit - d) / 10) throw std::runtime_error(err);
    value = value * 10 + d;
  }
  return value;
}

uint32_t u32_field(const Doc &doc, const char *name) {
  return static_cast<uint32_t>(parse_uint(
      doc.field(name), std::numeric_limits<uint32_t>::max(),
      doc.what + " manifest field is not an integer: " + name));
}

float positive_float_field(const Doc &doc, const char *name) {
  const Json &v = doc.field(name);
  const std::string err =
      doc.what + " manifest field is not a positive float: " + name;
  if (v.kind != Json::kNumber) throw std::runtime_error(err);
  errno = 0;
  char *end = nullptr;
  const float value = std::strtof(v.text.c_str(), &end);
  if (end == v.text.c_str() || *end != '\0' || errno == ERANGE || !(value > 0.0f))
    throw std::runtime_error(err);
  return value;
}

Doc parse_manifest(const std::string &path, const std::string &what,
                   uint32_t version, const char *format) {
  if (path.empty()) throw std::invalid_argument(what + " manifest path is empty");
  const std::vector<unsigned char> bytes = read_file(path, what);
  Doc doc{Parser(std::string(bytes.begin(), bytes.end())).parse(), what};
  if (doc.root.kind != Json::kObject)
    throw std::runtime_error(what + " manifest is not a JSON object");
  if (u32_field(doc, "version") != version)
    throw std::runtime_error("unsupported " + what + " manifest version");
  const std::string fmt = doc.str("format");
  if (fmt != format)
    throw std::runtime_error("unsupported " + what + " manifest format: " + fmt);
  const std::string dtype = doc.str("dtype");
  if (dtype != "f32")
    throw std::runtime_error("unsupported " + what + " dtype: " + dtype);
  return doc;
}

// Finds the unique tensor entry `name`, validates count and range, and copies
// it; returns the end offset in bytes.
uint64_t copy_tensor(const Doc &doc, const std::vector<unsigned char> &data,
                     const char *name, size_t count, std::vector<float> *out) {
  const Json &tensors = doc.field("tensors");
  if (tensors.kind != Json::kArray)
    throw std::runtime_error(doc.what + " manifest field is not an array: tensors");
  const Json *entry = nullptr;
  for (const Json &t : tensors.items) {
    const Json *n = t.kind == Json::kObject ? t.get("name") : nullptr;
    if (n && n->kind == Json::kString && n->text == name) {
      if (entry) throw std::runtime_error("duplicate " + doc.what + " tensor: " + name);
      entry = &t;
    }
  }
  if (!entry) throw std::runtime_error("missing " + doc.what + " tensor: " + name);
  const std::string tag = doc.what + " tensor '" + name + "'";
  const Json *off = entry->get("offset");
  const Json *cnt = entry->get("count");
  if (!off) throw std::runtime_error(tag + " is missing field: offset");
  if (!cnt) throw std::runtime_error(tag + " is missing field: count");
  const uint64_t offset = parse_uint(*off, std::numeric_limits<uint64_t>::max(),
                                     tag + " field is not an integer: offset");
  const uint64_t n = parse_uint(*cnt, std::numeric_limits<uint64_t>::max(),
                                tag + " field is not an integer: count");
  if (n != count) throw std::runtime_error(tag + " has unexpected count");
  const uint64_t bytes = checked_mul(count, sizeof(float), name);
  if (offset > std::numeric_limits<uint64_t>::max() - bytes)
    throw std::runtime_error(tag + " overflows offset");
  if (offset + bytes > data.size()) throw std::runtime_error(tag + " is out of range");
  out->resize(count);
  if (bytes) std::memcpy(out->data(), data.data() + offset, bytes);
  return offset + bytes;
}

void validate_shape(const LayerShape &s) {
  if (s.keys == 0 || s.hidden == 0 || s.heads == 0 || s.kv_heads == 0 ||
      s.head_dim == 0 || s.head_dim % 2 != 0 || s.intermediate == 0)
    throw std::runtime_error("mini decoder weight manifest has invalid shape");
  if (s.kv_heads > s.heads || s.heads % s.kv_heads != 0)
    throw std::runtime_error("mini decoder weight manifest has invalid GQA shape");
  if (s.heads > std::numeric_limits<uint32_t>::max() / s.head_dim)
    throw std::overflow_error("mini decoder q dimension overflows uint32");
}

void append(std::ofstream &data, std::ostream &manifest, const char *name,
            const std::vector<float> &values, uint64_t *offset, bool *first) {
  if (!*first) manifest << ",\n";
  *first = false;
  manifest << "    {\"name\":\"" << name << "\",\"offset\":" << *offset
           << ",\"count\":" << values.size() << "}";
  const size_t bytes = checked_mul(values.size(), sizeof(float), name);
  if (bytes) {
    data.write(reinterpret_cast<const char *>(values.data()),
               static_cast<std::streamsize>(bytes));
    if (!data)
      throw std::runtime_error(std::string("failed to write weight tensor: ") + name);
  }
  *offset += bytes;
}

}  // namespace

size_t layer_tensor_count(const LayerShape &s, int tensor) {
  const size_t h = s.hidden, q = size_t(s.heads) * s.head_dim,
               kv = size_t(s.kv_heads) * s.head_dim, i = s.intermediate;
  switch (tensor) {
    case kAttnNorm:
    case kMlpNorm:
      return h;
    case kQW:
      return checked_mul(q, h, "q_weight");
    case kKW:
      return checked_mul(kv, h, "k_weight");
    case kVW:
      return checked_mul(kv, h, "v_weight");
    case kQB:
      return q;
    case kKB:
    case kVB:
      return kv;
    case kOW:
      return checked_mul(h, q, "out_weight");
    case kGateW:
      return checked_mul(i, h, "gate_weight");
    case kUpW:
      return checked_mul(i, h, "up_weight");
    case kDownW:
      return checked_mul(h, i, "down_weight");
  }
  return 0;
}

LayerWeights load_layer(const std::string &manifest) {
  const Doc doc = parse_manifest(manifest, "mini decoder weight", 2,
                                 "lrrt.mini_decoder_weights");
  LayerWeights w;
  w.shape.keys = u32_field(doc, "keys");
  w.shape.hidden = u32_field(doc, "hidden");
  w.shape.heads = u32_field(doc, "heads");
  w.shape.head_dim = u32_field(doc, "head_dim");
  w.shape.intermediate = u32_field(doc, "intermediate");
  w.shape.kv_heads =
      doc.root.get("kv_heads") ? u32_field(doc, "kv_heads") : w.shape.heads;
  if (doc.root.get("rope_theta")) w.rope_theta = positive_float_field(doc, "rope_theta");
  validate_shape(w.shape);
  const std::vector<unsigned char> data = read_file(
      data_path(manifest, doc.str("data"), "mini decoder weight"),
      "mini decoder weight");
  uint64_t extent = 0;
  for (int t = 0; t < kLayerTensorCount; ++t) {
    extent = std::max(extent, copy_tensor(doc, data, kLayerTensorNames[t],
                                          layer_tensor_count(w.shape, t),
                                          &w.tensors[t]));
  }
  if (extent != data.size())
    throw std::runtime_error("mini decoder weight data size mismatch");
  return w;
}

TailWeights load_tail(const std::string &manifest) {
  const Doc doc = parse_manifest(manifest, "mini model tail", 1,
                                 "lrrt.mini_model_tail_weights");
  TailWeights w;
  w.hidden = u32_field(doc, "hidden");
  w.vocab = u32_field(doc, "vocab");
  const Json &ids = doc.field("token_ids");
  if (ids.kind != Json::kArray)
    throw std::runtime_error("mini model tail manifest field is not an array: token_ids");
  for (const Json &id : ids.items) {
    w.token_ids.push_back(static_cast<uint32_t>(parse_uint(
        id, std::numeric_limits<uint32_t>::max(),
        "mini model tail manifest array contains a non-integer: token_ids")));
  }
  if (w.hidden == 0 || w.vocab == 0 || w.token_ids.empty())
    throw std::runtime_error("mini model tail manifest has invalid shape");
  for (uint32_t id : w.token_ids)
    if (id >= w.vocab)
      throw std::runtime_error("mini model tail manifest has invalid token id");
  const std::vector<unsigned char> data = read_file(
      data_path(manifest, doc.str("data"), "mini model tail"), "mini model tail");
  uint64_t extent = 0;
  extent = std::max(extent, copy_tensor(doc, data, "token_embeddings",
                                        checked_mul(w.token_ids.size(), w.hidden,
                                                    "token_embeddings"),
                                        &w.token_embeddings));
  extent = std::max(extent, copy_tensor(doc, data, "final_norm_weight", w.hidden,
                                        &w.final_norm_weight));
  extent = std::max(extent, copy_tensor(doc, data, "lm_head_weight",
                                        checked_mul(w.vocab, w.hidden, "lm_head_weight"),
                                        &w.lm_head_weight));
  if (extent != data.size())
    throw std::runtime_error("mini model tail data size mismatch");
  return w;
}

void write_layer(const std::string &manifest_path, const std::string &data_name,
                 const LayerWeights &w) {
  if (manifest_path.empty() || data_name.empty())
    throw std::invalid_argument("mini decoder weight output path is empty");
  validate_shape(w.shape);
  if (!(w.rope_theta > 0.0f))
    throw std::runtime_error("mini decoder weights have invalid tensor sizes");
  for (int t = 0; t < kLayerTensorCount; ++t)
    if (w.tensors[t].size() != layer_tensor_count(w.shape, t))
      throw std::runtime_error("mini decoder weights have invalid tensor sizes");
  const std::string path = data_path(manifest_path, data_name, "mini decoder weight");
  std::ofstream data(path, std::ios::binary | std::ios::trunc);
  if (!data) throw std::runtime_error("failed to create mini decoder weight data file: " + path);
  std::ofstream manifest(manifest_path, std::ios::binary | std::ios::trunc);
  if (!manifest)
    throw std::runtime_error("failed to create mini decoder weight manifest: " + manifest_path);
  manifest << "{\n"
           << "  \"format\": \"lrrt.mini_decoder_weights\",\n"
           << "  \"version\": 2,\n"
           << "  \"dtype\": \"f32\",\n"
           << "  \"data\": \"" << data_name << "\",\n"
           << "  \"keys\": " << w.shape.keys << ",\n"
           << "  \"hidden\": " << w.shape.hidden << ",\n"
           << "  \"heads\": " << w.shape.heads << ",\n"
           << "  \"kv_heads\": " << w.shape.kv_heads << ",\n"
           << "  \"head_dim\": " << w.shape.head_dim << ",\n"
           << "  \"intermediate\": " << w.shape.intermediate << ",\n"
           << "  \"rope_theta\": " << w.rope_theta << ",\n"
           << "  \"tensors\": [\n";
  uint64_t offset = 0;
  bool first = true;
  for (int t = 0; t < kLayerTensorCount; ++t)
    append(data, manifest, kLayerTensorNames[t], w.tensors[t], &offset, &first);
  manifest << "\n  ]\n}\n";
  if (!manifest) throw std::runtime_error("failed to write mini decoder weight manifest");
}

void write_tail(const std::string &manifest_path, const std::string &data_name,
                const TailWeights &w) {
  if (manifest_path.empty() || data_name.empty())
    throw std::invalid_argument("mini model tail output path is empty");
  if (w.hidden == 0 || w.vocab == 0 || w.token_ids.empty() ||
      w.token_embeddings.size() != w.token_ids.size() * size_t(w.hidden) ||
      w.final_norm_weight.size() != w.hidden ||
      w.lm_head_weight.size() != size_t(w.vocab) * w.hidden)
    throw std::runtime_error("mini model tail weights have invalid sizes");
  for (uint32_t id : w.token_ids)
    if (id >= w.vocab) throw std::runtime_error("mini model tail weights have invalid token id");
  const std::string path = data_path(manifest_path, data_name, "mini model tail");
  std::ofstream data(path, std::ios::binary | std::ios::trunc);
  if (!data) throw std::runtime_error("failed to create mini model tail data file: " + path);
  std::ofstream manifest(manifest_path, std::ios::binary | std::ios::trunc);
  if (!manifest)
    throw std::runtime_error("failed to create mini model tail manifest: " + manifest_path);
  manifest << "{\n"
           << "  \"format\": \"lrrt.mini_model_tail_weights\",\n"
           << "  \"version\": 1,\n"
           << "  \"dtype\": \"f32\",\n"
           << "  \"data\": \"" << data_name << "\",\n"
           << "  \"hidden\": " << w.hidden << ",\n"
           << "  \"vocab\": " << w.vocab << ",\n"
           << "  \"token_ids\": [";
  for (size_t i = 0; i < w.token_ids.size(); ++i) {
    if (i) manifest << ", ";
    manifest << w.token_ids[i];
  }
  manifest << "],\n  \"tensors\": [\n";
  uint64_t offset = 0;
  bool first = true;
  append(data, manifest, "token_embeddings", w.token_embeddings, &offset, &first);
  append(data, manifest, "final_norm_weight", w.final_norm_weight, &offset, &first);
  append(data, manifest, "lm_head_weight", w.lm_head_weight, &offset, &first);
  manifest << "\n  ]\n}\n";
  if (!manifest) throw std::runtime_error("failed to write mini model tail manifest");
}

}  // namespace qd::bundle
