// safetensors.cpp — safetensors reading and writing, the HF key mappers, and
// the PEFT-format LoRA saver/loader of the operators library.
#include <algorithm>
#include <cctype>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <sstream>
#include <stdexcept>

#include "finetune_ops/graph/lora_saver.h"
#include "finetune_ops/graph/safetensors_loader.h"
#include "mft_engine.h"

namespace ops {

namespace {

// ------------------------------------------------------------------ JSON --
// The subset a safetensors header needs: objects (member order kept),
// arrays, strings with escapes, numbers (raw text kept for exact uint64),
// true / false / null.
struct JVal {
  enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
  bool b = false;
  std::string text;  // string value, or the number's literal
  std::vector<JVal> arr;
  std::vector<std::pair<std::string, JVal>> obj;
};

class JParser {
 public:
  explicit JParser(const std::string& s) : s_(s) {}
  JVal parse_document() {
    JVal v = value(0);
    ws();
    if (p_ != s_.size()) fail("trailing characters");
    return v;
  }

 private:
  [[noreturn]] void fail(const char* what) const {
    throw std::runtime_error(std::string("safetensors header: ") + what + " at byte " + std::to_string(p_));
  }
  void ws() {
    while (p_ < s_.size() && (s_[p_] == ' ' || s_[p_] == '\t' || s_[p_] == '\n' || s_[p_] == '\r')) ++p_;
  }
  bool lit(const char* w) {
    const size_t n = std::strlen(w);
    if (s_.compare(p_, n, w) != 0) return false;
    p_ += n;
    return true;
  }
  static void utf8(std::string& out, uint32_t cp) {
    if (cp < 0x80) {
      out += char(cp);
    } else if (cp < 0x800) {
      out += char(0xC0 | (cp >> 6));
      out += char(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      out += char(0xE0 | (cp >> 12));
      out += char(0x80 | ((cp >> 6) & 0x3F));
      out += char(0x80 | (cp & 0x3F));
    } else {
      out += char(0xF0 | (cp >> 18));
      out += char(0x80 | ((cp >> 12) & 0x3F));
      out += char(0x80 | ((cp >> 6) & 0x3F));
      out += char(0x80 | (cp & 0x3F));
    }
  }
  uint32_t hex4() {
    if (p_ + 4 > s_.size()) fail("short \\u escape");
    uint32_t v = 0;
    for (int i = 0; i < 4; ++i) {
      const char c = s_[p_++];
      v <<= 4;
      if (c >= '0' && c <= '9') v |= c - '0';
      else if (c >= 'a' && c <= 'f') v |= c - 'a' + 10;
      else if (c >= 'A' && c <= 'F') v |= c - 'A' + 10;
      else fail("bad \\u escape");
    }
    return v;
  }
  std::string str() {
    if (p_ >= s_.size() || s_[p_] != '"') fail("string expected");
    ++p_;
    std::string out;
    while (true) {
      if (p_ >= s_.size()) fail("unterminated string");
      const char c = s_[p_++];
      if (c == '"') return out;
      if ((unsigned char)c < 0x20) fail("control character in string");
      if (c != '\\') {
        out += c;
        continue;
      }
      if (p_ >= s_.size()) fail("unterminated escape");
      const char e = s_[p_++];
      switch (e) {
        case '"': out += '"'; break;
        case '\\': out += '\\'; break;
        case '/': out += '/'; break;
        case 'b': out += '\b'; break;
        case 'f': out += '\f'; break;
        case 'n': out += '\n'; break;
        case 'r': out += '\r'; break;
        case 't': out += '\t'; break;
        case 'u': {
          uint32_t cp = hex4();
          if (cp >= 0xD800 && cp < 0xDC00) {  // surrogate pair
            if (!lit("\\u")) fail("lone high surrogate");
            const uint32_t lo = hex4();
            if (lo < 0xDC00 || lo >= 0xE000) fail("bad low surrogate");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          utf8(out, cp);
          break;
        }
        default: fail("bad escape");
      }
    }
  }
  JVal value(int depth) {
    if (depth > 64) fail("nesting too deep");
    ws();
    if (p_ >= s_.size()) fail("value expected");
    JVal v;
    const char c = s_[p_];
    if (c == '{') {
      v.kind = JVal::Obj;
      ++p_;
      ws();
      if (p_ < s_.size() && s_[p_] == '}') {
        ++p_;
        return v;
      }
      while (true) {
        ws();
        std::string k = str();
        ws();
        if (p_ >= s_.size() || s_[p_] != ':') fail("':' expected");
        ++p_;
        v.obj.emplace_back(std::move(k), value(depth + 1));
        ws();
        if (p_ < s_.size() && s_[p_] == ',') {
          ++p_;
          continue;
        }
        if (p_ < s_.size() && s_[p_] == '}') {
          ++p_;
          return v;
        }
        fail("',' or '}' expected");
      }
    }
    if (c == '[') {
      v.kind = JVal::Arr;
      ++p_;
      ws();
      if (p_ < s_.size() && s_[p_] == ']') {
        ++p_;
        return v;
      }
      while (true) {
        v.arr.push_back(value(depth + 1));
        ws();
        if (p_ < s_.size() && s_[p_] == ',') {
          ++p_;
          continue;
        }
        if (p_ < s_.size() && s_[p_] == ']') {
          ++p_;
          return v;
        }
        fail("',' or ']' expected");
      }
    }
    if (c == '"') {
      v.kind = JVal::Str;
      v.text = str();
      return v;
    }
    if (lit("true")) {
      v.kind = JVal::Bool;
      v.b = true;
      return v;
    }
    if (lit("false")) {
      v.kind = JVal::Bool;
      return v;
    }
    if (lit("null")) return v;
    const size_t b = p_;
    if (p_ < s_.size() && s_[p_] == '-') ++p_;
    while (p_ < s_.size() && (std::isdigit((unsigned char)s_[p_]) || s_[p_] == '.' || s_[p_] == 'e' ||
                              s_[p_] == 'E' || s_[p_] == '+' || s_[p_] == '-'))
      ++p_;
    if (p_ == b) fail("unexpected character");
    v.kind = JVal::Num;
    v.text = s_.substr(b, p_ - b);
    return v;
  }
  const std::string& s_;
  size_t p_ = 0;
};

// A non-negative integer literal as uint64 (no sign, fraction or exponent).
uint64_t as_u64(const JVal& v, const char* what) {
  if (v.kind != JVal::Num || v.text.empty()) throw std::runtime_error(std::string("safetensors header: ") + what);
  uint64_t x = 0;
  for (char c : v.text) {
    if (c < '0' || c > '9') throw std::runtime_error(std::string("safetensors header: ") + what);
    if (x > (UINT64_MAX - 9) / 10) throw std::runtime_error(std::string("safetensors header: overflow in ") + what);
    x = x * 10 + (c - '0');
  }
  return x;
}

const JVal* member(const JVal& o, const char* key) {
  for (const auto& kv : o.obj)
    if (kv.first == key) return &kv.second;
  return nullptr;
}

// Bytes per element of a safetensors dtype, 0 if unknown.
size_t st_dtype_size(const std::string& d) {
  if (d == "F64" || d == "I64" || d == "U64") return 8;
  if (d == "F32" || d == "I32" || d == "U32") return 4;
  if (d == "F16" || d == "BF16" || d == "I16" || d == "U16") return 2;
  if (d == "I8" || d == "U8" || d == "BOOL" || d == "F8_E4M3" || d == "F8_E5M2") return 1;
  return 0;
}

std::string json_escape(const std::string& s) {
  std::string o;
  for (unsigned char c : s) {
    if (c == '"') o += "\\\"";
    else if (c == '\\') o += "\\\\";
    else if (c < 0x20) {
      char buf[8];
      std::snprintf(buf, sizeof buf, "\\u%04x", c);
      o += buf;
    } else {
      o += char(c);
    }
  }
  return o;
}

bool starts_with(const std::string& s, const std::string& p) { return s.compare(0, p.size(), p) == 0; }
bool ends_with(const std::string& s, const std::string& p) {
  return s.size() >= p.size() && s.compare(s.size() - p.size(), p.size(), p) == 0;
}

// IEEE binary16 → binary32, exact (subnormals normalised, Inf/NaN kept).
float half_to_float(uint16_t h) {
  const uint32_t sign = uint32_t(h >> 15) << 31;
  uint32_t exp = (h >> 10) & 0x1F, man = h & 0x3FF, bits;
  if (exp == 0x1F) {
    bits = sign | 0x7F800000u | (man << 13);
  } else if (exp != 0) {
    bits = sign | ((exp + 112) << 23) | (man << 13);
  } else if (man == 0) {
    bits = sign;
  } else {  // subnormal: man·2^-24, shifted up to an implicit leading one
    int e = -1;
    do {
      man <<= 1;
      ++e;
    } while (!(man & 0x400));
    bits = sign | (uint32_t(112 - e) << 23) | ((man & 0x3FF) << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

void transpose_bytes(HostTensor& h, size_t es) {
  if (h.shape.size() != 2) throw std::invalid_argument("safetensors: transpose of a tensor that is not 2-D: " + h.name);
  const int64_t rows = h.shape[0], cols = h.shape[1];
  std::vector<uint8_t> out(h.bytes.size());
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < cols; ++c) std::memcpy(&out[(c * rows + r) * es], &h.bytes[(r * cols + c) * es], es);
  h.bytes.swap(out);
  h.shape = {cols, rows};
}

bool is_embedding(const std::string& name) {
  return name.find("wte") != std::string::npos || name.find("wpe") != std::string::npos ||
         name.find("embed") != std::string::npos || name.find("lm_head") != std::string::npos;
}

TensorPtr to_gpu(const HostTensor& h) {
  return std::make_shared<Tensor>(h.shape, static_cast<const void*>(h.bytes.data()), h.dtype, kGPU);
}

}  // namespace

// ---------------------------------------------------------------- reader --

SafeTensorsReader::SafeTensorsReader(const std::string& path) : path_(path) {}

void SafeTensorsReader::parse_header() {
  if (parsed_) return;
  std::ifstream f(path_, std::ios::binary);
  if (!f) throw std::runtime_error("SafeTensorsReader: cannot open " + path_);
  f.seekg(0, std::ios::end);
  const uint64_t file_size = (uint64_t)f.tellg();
  f.seekg(0);
  if (file_size < 8) throw std::runtime_error("SafeTensorsReader: file too short: " + path_);
  unsigned char len8[8];
  f.read(reinterpret_cast<char*>(len8), 8);
  uint64_t n = 0;
  for (int i = 7; i >= 0; --i) n = (n << 8) | len8[i];
  if (n > (100u << 20) || 8 + n > file_size)
    throw std::runtime_error("SafeTensorsReader: bad header length " + std::to_string(n) + " in " + path_);
  std::string hdr(n, '\0');
  f.read(&hdr[0], (std::streamsize)n);
  if (!f) throw std::runtime_error("SafeTensorsReader: short read of the header of " + path_);
  const JVal root = JParser(hdr).parse_document();
  if (root.kind != JVal::Obj) throw std::runtime_error("safetensors header: not an object");
  data_start_ = 8 + n;
  data_len_ = file_size - data_start_;
  for (const auto& kv : root.obj) {
    if (kv.first == "__metadata__") {
      if (kv.second.kind != JVal::Obj) throw std::runtime_error("safetensors header: __metadata__ not an object");
      for (const auto& m : kv.second.obj) {
        if (m.second.kind != JVal::Str) throw std::runtime_error("safetensors header: metadata value not a string");
        metadata_[m.first] = m.second.text;
      }
      continue;
    }
    const JVal& t = kv.second;
    const JVal* dt = t.kind == JVal::Obj ? member(t, "dtype") : nullptr;
    const JVal* sh = t.kind == JVal::Obj ? member(t, "shape") : nullptr;
    const JVal* off = t.kind == JVal::Obj ? member(t, "data_offsets") : nullptr;
    if (!dt || dt->kind != JVal::Str || !sh || sh->kind != JVal::Arr || !off || off->kind != JVal::Arr ||
        off->arr.size() != 2)
      throw std::runtime_error("safetensors header: malformed entry " + kv.first);
    SafeTensorInfo info;
    info.dtype = dt->text;
    uint64_t numel = 1;
    for (const auto& d : sh->arr) {
      const uint64_t x = as_u64(d, "shape");
      if (x && numel > UINT64_MAX / x) throw std::runtime_error("safetensors header: shape overflow in " + kv.first);
      numel *= x;
      info.shape.push_back((int64_t)x);
    }
    info.begin = as_u64(off->arr[0], "data_offsets");
    info.end = as_u64(off->arr[1], "data_offsets");
    const size_t es = st_dtype_size(info.dtype);
    if (!es) throw std::runtime_error("safetensors header: unknown dtype " + info.dtype + " of " + kv.first);
    if (info.begin > info.end || info.end > data_len_ || info.end - info.begin != numel * es)
      throw std::runtime_error("safetensors header: data_offsets of " + kv.first + " do not match its dtype, shape "
                               "and the file size");
    tensors_[kv.first] = std::move(info);
  }
  parsed_ = true;
}

std::vector<std::string> SafeTensorsReader::get_tensor_names() {
  parse_header();
  std::vector<std::string> out;
  for (const auto& kv : tensors_) out.push_back(kv.first);
  return out;
}

bool SafeTensorsReader::has_tensor(const std::string& key) {
  parse_header();
  try {
    resolve(key);
    return true;
  } catch (const std::runtime_error&) {
    return false;
  }
}

const SafeTensorInfo& SafeTensorsReader::tensor_info(const std::string& key) { return tensors_.at(resolve(key)); }

const std::map<std::string, std::string>& SafeTensorsReader::metadata() {
  parse_header();
  return metadata_;
}

std::string SafeTensorsReader::resolve(const std::string& key) {
  parse_header();
  if (tensors_.count(key)) return key;
  static const char* const kPrefixes[] = {"transformer.", "model.", "language_model.model.", "language_model."};
  for (const char* p : kPrefixes) {
    if (tensors_.count(p + key)) return p + key;
    if (starts_with(key, p) && tensors_.count(key.substr(std::strlen(p)))) return key.substr(std::strlen(p));
  }
  throw std::runtime_error("SafeTensorsReader: tensor " + key + " not found in " + path_);
}

HostTensor SafeTensorsReader::read_host(const std::string& key, bool transpose) {
  const std::string k = resolve(key);
  const SafeTensorInfo& info = tensors_.at(k);
  std::ifstream f(path_, std::ios::binary);
  if (!f) throw std::runtime_error("SafeTensorsReader: cannot open " + path_);
  std::vector<uint8_t> raw(info.end - info.begin);
  f.seekg((std::streamoff)(data_start_ + info.begin));
  f.read(reinterpret_cast<char*>(raw.data()), (std::streamsize)raw.size());
  if (!f) throw std::runtime_error("SafeTensorsReader: short read of " + k);
  HostTensor h;
  h.name = key;
  h.shape = info.shape;
  if (info.dtype == "F32") {
    h.dtype = kFloat32;
    h.bytes.swap(raw);
  } else if (info.dtype == "F16") {
    h.dtype = kFloat16;
    h.bytes.swap(raw);
  } else if (info.dtype == "BF16") {  // bf16 is the top half of an fp32
    h.dtype = kFloat32;
    h.bytes.resize(raw.size() * 2);
    for (size_t i = 0; i < raw.size() / 2; ++i) {
      h.bytes[4 * i + 0] = 0;
      h.bytes[4 * i + 1] = 0;
      h.bytes[4 * i + 2] = raw[2 * i];
      h.bytes[4 * i + 3] = raw[2 * i + 1];
    }
  } else {
    throw std::runtime_error("SafeTensorsReader: dtype " + info.dtype + " of " + k + " is not a float type");
  }
  if (transpose) transpose_bytes(h, h.dtype == kFloat16 ? 2 : 4);
  return h;
}

std::vector<HostTensor> SafeTensorsReader::read_mapped_host(
    const std::unordered_map<std::string, std::string>& internal_to_hf, const SafeTensorsLoadOptions& opts) {
  parse_header();
  std::map<std::string, std::string> ordered(internal_to_hf.begin(), internal_to_hf.end());
  std::vector<HostTensor> out;
  out.reserve(ordered.size());
  for (const auto& kv : ordered) {
    const SafeTensorInfo& info = tensor_info(kv.second);
    const bool tr = opts.transpose_linear && info.shape.size() == 2 && !is_embedding(kv.first);
    HostTensor h = read_host(kv.second, tr);
    h.name = kv.first;
    if (opts.verbose) {
      std::printf("  [safetensors] %s <- %s %s [", kv.first.c_str(), kv.second.c_str(), info.dtype.c_str());
      for (size_t i = 0; i < h.shape.size(); ++i) std::printf(i ? ",%lld" : "%lld", (long long)h.shape[i]);
      std::printf("]%s\n", tr ? " (transposed)" : "");
    }
    out.push_back(std::move(h));
  }
  return out;
}

TensorPtr SafeTensorsReader::load_tensor(const std::string& key, bool transpose) {
  return to_gpu(read_host(key, transpose));
}

std::unordered_map<std::string, TensorPtr> SafeTensorsReader::load_tensors_mapped(
    const std::unordered_map<std::string, std::string>& internal_to_hf, const SafeTensorsLoadOptions& opts) {
  std::unordered_map<std::string, TensorPtr> out;
  for (auto& h : read_mapped_host(internal_to_hf, opts)) out[h.name] = to_gpu(h);
  return out;
}

// ---------------------------------------------------------------- writer --

void write_safetensors(const std::string& path, const std::vector<SafeTensorsEntry>& entries,
                       const std::map<std::string, std::string>& metadata) {
  std::ostringstream hdr;
  hdr << "{";
  bool first = true;
  if (!metadata.empty()) {
    hdr << "\"__metadata__\":{";
    bool f2 = true;
    for (const auto& kv : metadata) {
      hdr << (f2 ? "" : ",") << "\"" << json_escape(kv.first) << "\":\"" << json_escape(kv.second) << "\"";
      f2 = false;
    }
    hdr << "}";
    first = false;
  }
  uint64_t off = 0;
  for (const auto& e : entries) {
    const size_t es = st_dtype_size(e.dtype);
    if (!es) throw std::invalid_argument("write_safetensors: unknown dtype " + e.dtype);
    uint64_t numel = 1;
    for (auto d : e.shape) {
      if (d < 0) throw std::invalid_argument("write_safetensors: negative dimension in " + e.name);
      numel *= (uint64_t)d;
    }
    if (numel * es != e.nbytes || (e.nbytes && !e.data))
      throw std::invalid_argument("write_safetensors: " + e.name + " has " + std::to_string(e.nbytes) +
                                  " bytes, dtype and shape need " + std::to_string(numel * es));
    hdr << (first ? "" : ",") << "\"" << json_escape(e.name) << "\":{\"dtype\":\"" << e.dtype << "\",\"shape\":[";
    for (size_t i = 0; i < e.shape.size(); ++i) hdr << (i ? "," : "") << e.shape[i];
    hdr << "],\"data_offsets\":[" << off << "," << off + e.nbytes << "]}";
    off += e.nbytes;
    first = false;
  }
  hdr << "}";
  std::string h = hdr.str();
  while ((8 + h.size()) % 8) h += ' ';
  const auto parent = std::filesystem::path(path).parent_path();
  if (!parent.empty()) std::filesystem::create_directories(parent);
  std::ofstream f(path, std::ios::binary);
  if (!f) throw std::runtime_error("write_safetensors: cannot open " + path + " for writing");
  unsigned char len8[8];
  for (int i = 0; i < 8; ++i) len8[i] = (unsigned char)(((uint64_t)h.size() >> (8 * i)) & 0xFF);
  f.write(reinterpret_cast<const char*>(len8), 8);
  f.write(h.data(), (std::streamsize)h.size());
  for (const auto& e : entries) f.write(static_cast<const char*>(e.data), (std::streamsize)e.nbytes);
  if (!f) throw std::runtime_error("write_safetensors: write failed for " + path);
}

// ----------------------------------------------------------- key mappers --

std::unordered_map<std::string, std::string> GPT2KeyMapper::generate_gpt2_mapping(int n_layer) {
  static const char* const kBlock[][2] = {
      {"ln_1.weight", "ln_1.weight"},           {"ln_1.bias", "ln_1.bias"},
      {"attn.qkv.weight", "attn.c_attn.weight"}, {"attn.qkv.bias", "attn.c_attn.bias"},
      {"attn.proj.weight", "attn.c_proj.weight"}, {"attn.proj.bias", "attn.c_proj.bias"},
      {"ln_2.weight", "ln_2.weight"},           {"ln_2.bias", "ln_2.bias"},
      {"mlp.fc_in.weight", "mlp.c_fc.weight"},   {"mlp.fc_in.bias", "mlp.c_fc.bias"},
      {"mlp.fc_out.weight", "mlp.c_proj.weight"}, {"mlp.fc_out.bias", "mlp.c_proj.bias"}};
  std::unordered_map<std::string, std::string> m;
  m["wte.weight"] = "wte.weight";
  m["wpe.weight"] = "wpe.weight";
  for (int i = 0; i < n_layer; ++i)
    for (const auto& kv : kBlock)
      m["blocks." + std::to_string(i) + "." + kv[0]] = "h." + std::to_string(i) + "." + kv[1];
  m["ln_f.weight"] = "ln_f.weight";
  m["ln_f.bias"] = "ln_f.bias";
  return m;
}

namespace {
std::unordered_map<std::string, std::string> hf_decoder_mapping(int n_layer, bool gemma) {
  std::vector<std::string> per_layer = {"input_layernorm.weight",        "self_attn.q_proj.weight",
                                        "self_attn.k_proj.weight",       "self_attn.v_proj.weight",
                                        "self_attn.o_proj.weight",       "post_attention_layernorm.weight",
                                        "mlp.gate_proj.weight",          "mlp.up_proj.weight",
                                        "mlp.down_proj.weight"};
  if (gemma) {
    for (const char* s : {"self_attn.q_norm.weight", "self_attn.k_norm.weight", "pre_feedforward_layernorm.weight",
                          "post_feedforward_layernorm.weight"})
      per_layer.push_back(s);
  } else {
    for (const char* s : {"self_attn.q_proj.bias", "self_attn.k_proj.bias", "self_attn.v_proj.bias"})
      per_layer.push_back(s);
  }
  std::unordered_map<std::string, std::string> m;
  m["embed_tokens.weight"] = "model.embed_tokens.weight";
  m["norm.weight"] = "model.norm.weight";
  for (int i = 0; i < n_layer; ++i)
    for (const auto& s : per_layer) {
      const std::string name = "layers." + std::to_string(i) + "." + s;
      m[name] = "model." + name;
    }
  return m;
}
}  // namespace

std::unordered_map<std::string, std::string> QwenKeyMapper::generate_qwen_mapping(int n_layer) {
  return hf_decoder_mapping(n_layer, false);
}

std::unordered_map<std::string, std::string> GemmaKeyMapper::generate_gemma_mapping(int n_layer) {
  return hf_decoder_mapping(n_layer, true);
}

// ------------------------------------------------------------ LoRA saver --

namespace {

const char* const kGpt2Modules[4] = {"attn.c_attn", "attn.c_proj", "mlp.c_fc", "mlp.c_proj"};
const char* const kGpt2TargetNames[4] = {"AttnQKV", "AttnProj", "MlpFcIn", "MlpFcOut"};
const char* const kHfModules[7] = {"self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
                                   "mlp.gate_proj",    "mlp.up_proj",      "mlp.down_proj"};
const char* const kHfTargetNames[7] = {"q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"};

// A parsed adapter key: engine parameter name, family (0 GPT-2, 1 HF decoder),
// layer, target bit, and whether it is lora_A.
struct LoraKey {
  std::string engine_name;
  int arch = -1, layer = -1, bit = -1;
  bool is_a = false;
};

bool parse_lora_key(const std::string& key, LoraKey& out) {
  std::string n = key;
  if (starts_with(n, "base_model.model.")) n = n.substr(17);
  if (ends_with(n, ".weight")) n = n.substr(0, n.size() - 7);
  bool is_a;
  if (ends_with(n, ".lora_A")) is_a = true;
  else if (ends_with(n, ".lora_B")) is_a = false;
  else return false;
  const std::string module_path = n.substr(0, n.size() - 7);
  std::string rest;
  int arch;
  if (starts_with(module_path, "transformer.h.") || starts_with(module_path, "h.")) {
    arch = 0;
    rest = module_path.substr(starts_with(module_path, "h.") ? 2 : 14);
  } else {
    std::string m = module_path;
    if (starts_with(m, "language_model.")) m = m.substr(15);
    if (starts_with(m, "model.")) m = m.substr(6);
    if (!starts_with(m, "layers.")) return false;
    arch = 1;
    rest = m.substr(7);
  }
  const size_t dot = rest.find('.');
  if (dot == std::string::npos || dot == 0) return false;
  int layer = 0;
  for (size_t i = 0; i < dot; ++i) {
    if (rest[i] < '0' || rest[i] > '9') return false;
    layer = layer * 10 + (rest[i] - '0');
    if (layer > 100000) return false;
  }
  const std::string mod = rest.substr(dot + 1);
  int bit = -1;
  const int nmod = arch == 0 ? 4 : 7;
  for (int b = 0; b < nmod; ++b)
    if (mod == (arch == 0 ? kGpt2Modules[b] : kHfModules[b])) bit = b;
  if (bit < 0) return false;
  out.arch = arch;
  out.layer = layer;
  out.bit = bit;
  out.is_a = is_a;
  out.engine_name = (arch == 0 ? "h." : "layers.") + std::to_string(layer) + "." + mod + (is_a ? ".lora_A" : ".lora_B");
  return true;
}

// (in, out) of the linear a target bit names.
std::pair<int64_t, int64_t> lora_dims(const EngineModelConfig& c, int bit) {
  const int64_t d = c.d, ff = c.d_ff;
  if (c.arch == MFT_ARCH_GPT2) {
    const std::pair<int64_t, int64_t> g[4] = {{d, 3 * d}, {d, d}, {d, ff}, {ff, d}};
    return g[bit];
  }
  const int64_t q = (int64_t)c.n_head * c.head_dim, kv = (int64_t)c.n_kv_head * c.head_dim;
  const std::pair<int64_t, int64_t> h[7] = {{d, q}, {d, kv}, {d, kv}, {q, d}, {d, ff}, {d, ff}, {ff, d}};
  return h[bit];
}

std::string fmt_float(float v) {
  char buf[32];
  std::snprintf(buf, sizeof buf, "%.9g", v);
  return buf;
}

void save_impl(const std::string& path, EngineModel& model, int rank, float alpha, float dropout, bool split_qkv) {
  if (!model.has_lora()) throw std::invalid_argument("LoraSaver: the model has no LoRA adapters attached");
  if (rank != model.lora_rank())
    throw std::invalid_argument("LoraSaver: spec rank " + std::to_string(rank) + " differs from the model's " +
                                std::to_string(model.lora_rank()));
  const bool gpt2 = model.engine_config().arch == MFT_ARCH_GPT2;
  const std::string prefix = gpt2 ? "base_model.model.transformer." : "base_model.model.model.";
  std::vector<SafeTensorsEntry> entries;
  std::vector<TensorPtr> keep;
  for (const auto& name : model.parameter_names()) {
    if (!ends_with(name, ".lora_A") && !ends_with(name, ".lora_B")) continue;
    TensorPtr t = model.get_parameter(name);
    keep.push_back(t);
    const float* host = static_cast<const Tensor&>(*t).data<float>();
    entries.push_back({prefix + name + ".weight", "F32", t->shape(), host, (size_t)t->numel() * 4});
  }
  const int mask = model.lora_mask();
  std::string targets, modules_json;
  const int nbits = gpt2 ? 4 : 7;
  for (int b = 0; b < nbits; ++b) {
    if (!((mask >> b) & 1)) continue;
    const std::string tn = gpt2 ? kGpt2TargetNames[b] : kHfTargetNames[b];
    // PEFT matches target_modules as a suffix of the module path; GPT-2's
    // two c_proj linears need their parent to tell them apart.
    const std::string pm = gpt2 ? (b == 0 ? "c_attn" : b == 2 ? "c_fc" : kGpt2Modules[b]) : kHfTargetNames[b];
    targets += (targets.empty() ? "" : ",") + tn;
    modules_json += std::string(modules_json.empty() ? "" : ", ") + "\"" + pm + "\"";
  }
  std::map<std::string, std::string> meta = {{"format", "pt"},
                                             {"lora_rank", std::to_string(rank)},
                                             {"lora_alpha", fmt_float(alpha)},
                                             {"lora_dropout", fmt_float(dropout)},
                                             {"split_qkv", split_qkv ? "true" : "false"},
                                             {gpt2 ? "targets" : "target_modules", targets},
                                             {"arch", gpt2 ? "gpt2" : "hf_decoder"}};
  write_safetensors(path, entries, meta);
  const std::filesystem::path p(path);
  if (p.filename() == "adapter_model.safetensors") {
    std::ofstream cfg(p.parent_path() / "adapter_config.json");
    if (!cfg) throw std::runtime_error("LoraSaver: cannot write adapter_config.json beside " + path);
    cfg << "{\n  \"peft_type\": \"LORA\",\n  \"task_type\": \"CAUSAL_LM\",\n  \"r\": " << rank
        << ",\n  \"lora_alpha\": " << fmt_float(alpha) << ",\n  \"lora_dropout\": " << fmt_float(dropout)
        << ",\n  \"target_modules\": [" << modules_json << "],\n  \"fan_in_fan_out\": " << (gpt2 ? "true" : "false")
        << ",\n  \"bias\": \"none\",\n  \"base_model_name_or_path\": \"\"\n}\n";
  }
}

// A numeric value of a top-level key in a small JSON file, or NAN.
float json_file_num(const std::string& path, const char* key) {
  std::ifstream f(path);
  if (!f) return NAN;
  std::stringstream ss;
  ss << f.rdbuf();
  try {
    const JVal root = JParser(ss.str()).parse_document();
    const JVal* v = root.kind == JVal::Obj ? member(root, key) : nullptr;
    if (v && v->kind == JVal::Num) return std::stof(v->text);
  } catch (const std::exception&) {
  }
  return NAN;
}

}  // namespace

void LoraSaver::save_safetensors(const std::string& path, EngineModel& model, const LoraSpec& spec) {
  if (model.engine_config().arch != MFT_ARCH_GPT2) throw std::invalid_argument("LoraSaver: LoraSpec is for GPT-2");
  int mask = 0;
  for (auto t : spec.targets) mask |= 1 << (int)t;
  if (mask != model.lora_mask()) throw std::invalid_argument("LoraSaver: spec targets differ from the model's adapters");
  save_impl(path, model, spec.rank, spec.alpha, spec.dropout, spec.split_qkv);
}

void LoraSaver::save_safetensors(const std::string& path, EngineModel& model, const GemmaLoraSpec& spec) {
  save_impl(path, model, spec.rank, spec.alpha, spec.dropout, false);
}

void LoraSaver::save_safetensors(const std::string& path, EngineModel& model) {
  save_impl(path, model, model.lora_rank(), model.lora_alpha(), model.lora_dropout(), false);
}

LoraState LoraSaver::load_safetensors(const std::string& path) {
  SafeTensorsReader r(path);
  r.parse_header();
  LoraState st;
  int mask = 0;
  for (const auto& name : r.get_tensor_names()) {
    LoraKey k;
    if (!parse_lora_key(name, k)) continue;
    if (st.arch >= 0 && st.arch != k.arch)
      throw std::runtime_error("LoraSaver: " + path + " mixes GPT-2 and decoder-layer adapters");
    st.arch = k.arch;
    HostTensor h = r.read_host(name, false);
    if (h.dtype == kFloat16) {  // adapters are trained in fp32
      std::vector<uint8_t> w(h.bytes.size() * 2);
      for (size_t i = 0; i < h.bytes.size() / 2; ++i) {
        uint16_t v;
        std::memcpy(&v, &h.bytes[2 * i], 2);
        const float f = half_to_float(v);
        std::memcpy(&w[4 * i], &f, 4);
      }
      h.bytes.swap(w);
      h.dtype = kFloat32;
    }
    if (h.shape.size() != 2) throw std::runtime_error("LoraSaver: adapter " + name + " is not 2-D");
    const int r_here = (int)(k.is_a ? h.shape[0] : h.shape[1]);
    if (st.rank && r_here != st.rank) throw std::runtime_error("LoraSaver: mixed ranks in " + path);
    st.rank = r_here;
    st.n_layer = std::max(st.n_layer, k.layer + 1);
    mask |= 1 << k.bit;
    st.tensors[name] = to_gpu(h);
  }
  if (st.tensors.empty()) throw std::runtime_error("LoraSaver: no LoRA adapters in " + path);
  const auto& md = r.metadata();
  auto get = [&](const char* key) -> const std::string* {
    auto it = md.find(key);
    return it == md.end() ? nullptr : &it->second;
  };
  if (auto* v = get("lora_alpha")) {
    st.alpha = std::stof(*v);
  } else {
    const float a = json_file_num((std::filesystem::path(path).parent_path() / "adapter_config.json").string(),
                                  "lora_alpha");
    st.alpha = std::isnan(a) ? (float)st.rank : a;
  }
  if (auto* v = get("lora_dropout")) st.dropout = std::stof(*v);
  if (auto* v = get("split_qkv")) st.split_qkv = *v == "true" || *v == "1";
  for (int b = 0; b < (st.arch == 0 ? 4 : 7); ++b) {
    if (!((mask >> b) & 1)) continue;
    if (st.arch == 0) st.targets.push_back((LoraTarget)b);
    else st.target_modules.push_back(kHfTargetNames[b]);
  }
  return st;
}

bool LoraState::compatible_with(const EngineModel& model) const {
  const EngineModelConfig& c = model.engine_config();
  if (rank <= 0 || tensors.empty() || arch != (c.arch == MFT_ARCH_GPT2 ? 0 : 1) || n_layer > c.n_layer) return false;
  int mask = 0;
  std::vector<int> seen;
  for (const auto& kv : tensors) {
    LoraKey k;
    if (!parse_lora_key(kv.first, k) || k.arch != arch) return false;
    const auto io = lora_dims(c, k.bit);
    const std::vector<int64_t> want = k.is_a ? std::vector<int64_t>{rank, io.first} : std::vector<int64_t>{io.second, rank};
    if (kv.second->shape() != want) return false;
    mask |= 1 << k.bit;
    seen.push_back((k.layer * 8 + k.bit) * 2 + (k.is_a ? 1 : 0));
  }
  // Adapters attach model-wide per target: every layer needs both matrices.
  std::sort(seen.begin(), seen.end());
  seen.erase(std::unique(seen.begin(), seen.end()), seen.end());
  return (int)seen.size() == 2 * __builtin_popcount(mask) * c.n_layer;
}

void LoraSaver::attach_from_state(EngineModel& model, const LoraState& state) {
  if (!state.compatible_with(model))
    throw std::invalid_argument("LoraSaver::attach_from_state: adapters do not fit this model (architecture, "
                                "layer count, shapes or missing layers)");
  int mask = 0;
  for (const auto& kv : state.tensors) {
    LoraKey k;
    parse_lora_key(kv.first, k);
    mask |= 1 << k.bit;
  }
  model.set_lora_dropout(state.dropout);
  model.set_lora(state.rank, state.alpha, mask);
  for (const auto& kv : state.tensors) {
    LoraKey k;
    parse_lora_key(kv.first, k);
    model.assign_weight(k.engine_name, kv.second);
  }
}

}  // namespace ops
