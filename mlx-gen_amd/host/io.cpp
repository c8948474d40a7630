// io.cpp — packed-snapshot I/O of the C++ host API: safetensors files and the config.json
// "quantization" block.
//
// safetensors layout: an 8-byte little-endian header length n, n bytes of JSON mapping each
// tensor name to {"dtype", "shape", "data_offsets": [begin, end]} (plus an optional
// "__metadata__" object of strings), then the raw little-endian tensor bytes.  Packed codes are
// stored as U32, as MLX writes them, so snapshots interchange with the reference
// (src/quant.rs:92-116; mlx-gen-flux/src/convert.rs:46-78).
#include <algorithm>
#include <cctype>
#include <cerrno>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <sstream>
#include <variant>

#include "../../include/mlxq.h"
#include "mlxq.hpp"

namespace mlxq {

namespace {

// ---- a small JSON value: enough for safetensors headers and config.json files ----------------
struct Json;
using JsonObject = std::vector<std::pair<std::string, Json>>;  // keeps key order
using JsonArray = std::vector<Json>;
struct Json {
  std::variant<std::nullptr_t, bool, int64_t, double, std::string, JsonArray, JsonObject> v;
  const Json* get(const std::string& key) const {
    if (auto* o = std::get_if<JsonObject>(&v))
      for (const auto& kv : *o)
        if (kv.first == key) return &kv.second;
    return nullptr;
  }
  void set(const std::string& key, Json value) {
    if (!std::holds_alternative<JsonObject>(v)) v = JsonObject{};
    auto& o = std::get<JsonObject>(v);
    for (auto& kv : o)
      if (kv.first == key) {
        kv.second = std::move(value);
        return;
      }
    o.emplace_back(key, std::move(value));
  }
};

[[noreturn]] void bad_json(const std::string& what) { throw Error(MLXQ_EINVAL, "json: " + what); }

// Nesting limit of the parser: safetensors headers and config files nest a few levels; a header
// of nested brackets is rejected instead of exhausting the stack.
constexpr int kMaxJsonDepth = 64;

int hex_digit(char c) {
  if (c >= '0' && c <= '9') return c - '0';
  if (c >= 'a' && c <= 'f') return c - 'a' + 10;
  if (c >= 'A' && c <= 'F') return c - 'A' + 10;
  return -1;
}

struct JsonParser {
  const std::string& s;
  size_t i = 0;
  int depth = 0;
  void ws() {
    while (i < s.size() && std::isspace((unsigned char)s[i])) ++i;
  }
  char peek() {
    ws();
    if (i >= s.size()) bad_json("unexpected end");
    return s[i];
  }
  void expect(char c) {
    if (peek() != c) bad_json(std::string("expected '") + c + "'");
    ++i;
  }
  std::string str() {
    expect('"');
    std::string out;
    while (true) {
      if (i >= s.size()) bad_json("unterminated string");
      char c = s[i++];
      if (c == '"') break;
      if (c != '\\') {
        out += c;
        continue;
      }
      if (i >= s.size()) bad_json("bad escape");
      c = s[i++];
      switch (c) {
        case '"': case '\\': case '/': out += c; break;
        case 'b': out += '\b'; break;
        case 'f': out += '\f'; break;
        case 'n': out += '\n'; break;
        case 'r': out += '\r'; break;
        case 't': out += '\t'; break;
        case 'u': {
          if (i + 4 > s.size()) bad_json("bad \\u escape");
          unsigned cp = 0;
          for (int k = 0; k < 4; ++k) {
            const int d = hex_digit(s[i + k]);
            if (d < 0) bad_json("bad \\u escape");
            cp = cp * 16 + (unsigned)d;
          }
          i += 4;
          if (cp < 0x80) out += (char)cp;  // config files here are ASCII; keep others as UTF-8
          else if (cp < 0x800) { out += (char)(0xc0 | (cp >> 6)); out += (char)(0x80 | (cp & 0x3f)); }
          else { out += (char)(0xe0 | (cp >> 12)); out += (char)(0x80 | ((cp >> 6) & 0x3f)); out += (char)(0x80 | (cp & 0x3f)); }
          break;
        }
        default: bad_json("bad escape");
      }
    }
    return out;
  }
  Json value() {
    const char c = peek();
    Json j;
    if ((c == '{' || c == '[') && ++depth > kMaxJsonDepth) bad_json("nested too deeply");
    if (c == '{') {
      ++i;
      JsonObject o;
      if (peek() == '}') { ++i; j.v = o; --depth; return j; }
      while (true) {
        std::string k = str();
        expect(':');
        o.emplace_back(std::move(k), value());
        if (peek() == ',') { ++i; continue; }
        expect('}');
        break;
      }
      j.v = std::move(o);
      --depth;
    } else if (c == '[') {
      ++i;
      JsonArray a;
      if (peek() == ']') { ++i; j.v = a; --depth; return j; }
      while (true) {
        a.push_back(value());
        if (peek() == ',') { ++i; continue; }
        expect(']');
        break;
      }
      j.v = std::move(a);
      --depth;
    } else if (c == '"') {
      j.v = str();
    } else if (s.compare(i, 4, "true") == 0) { i += 4; j.v = true; }
    else if (s.compare(i, 5, "false") == 0) { i += 5; j.v = false; }
    else if (s.compare(i, 4, "null") == 0) { i += 4; j.v = nullptr; }
    else {
      size_t e = i;
      bool frac = false;
      while (e < s.size() && (std::isdigit((unsigned char)s[e]) || strchr("+-.eE", s[e]))) {
        frac |= s[e] == '.' || s[e] == 'e' || s[e] == 'E';
        ++e;
      }
      if (e == i) bad_json("unexpected character");
      const std::string num = s.substr(i, e - i);
      i = e;
      char* end = nullptr;
      errno = 0;
      if (frac) {
        const double d = std::strtod(num.c_str(), &end);
        if (end != num.c_str() + num.size() || errno == ERANGE) bad_json("bad number " + num);
        j.v = d;
      } else {
        const long long n = std::strtoll(num.c_str(), &end, 10);
        if (end != num.c_str() + num.size() || errno == ERANGE) bad_json("bad integer " + num);
        j.v = (int64_t)n;
      }
    }
    return j;
  }
};

Json parse_json(const std::string& s) {
  JsonParser p{s};
  Json j = p.value();
  p.ws();
  if (p.i != s.size()) bad_json("trailing characters");
  return j;
}

void dump_json(const Json& j, std::string& out, int indent, int depth) {
  const std::string pad = indent ? std::string((depth + 1) * indent, ' ') : "";
  const std::string end = indent ? "\n" + std::string(depth * indent, ' ') : "";
  const char* sep = indent ? ",\n" : ",";
  if (std::holds_alternative<std::nullptr_t>(j.v)) out += "null";
  else if (auto* b = std::get_if<bool>(&j.v)) out += *b ? "true" : "false";
  else if (auto* n = std::get_if<int64_t>(&j.v)) out += std::to_string(*n);
  else if (auto* d = std::get_if<double>(&j.v)) {
    char buf[64];
    snprintf(buf, sizeof buf, "%.17g", *d);
    out += buf;
  } else if (auto* s = std::get_if<std::string>(&j.v)) {
    out += '"';
    for (char c : *s) {
      if (c == '"' || c == '\\') { out += '\\'; out += c; }
      else if (c == '\n') out += "\\n";
      else if ((unsigned char)c < 0x20) { char buf[8]; snprintf(buf, sizeof buf, "\\u%04x", c); out += buf; }
      else out += c;
    }
    out += '"';
  } else if (auto* a = std::get_if<JsonArray>(&j.v)) {
    out += '[';
    for (size_t k = 0; k < a->size(); ++k) {
      if (k) out += ",";
      dump_json((*a)[k], out, 0, 0);  // arrays inline (shapes, offsets)
    }
    out += ']';
  } else {
    const auto& o = std::get<JsonObject>(j.v);
    if (o.empty()) { out += "{}"; return; }
    out += indent ? "{\n" : "{";
    for (size_t k = 0; k < o.size(); ++k) {
      if (k) out += sep;
      out += pad;
      dump_json(Json{o[k].first}, out, 0, 0);
      out += indent ? ": " : ":";
      dump_json(o[k].second, out, indent, depth + 1);
    }
    out += end + "}";
  }
}

std::string read_file(const std::string& path) {
  std::ifstream f(path, std::ios::binary);
  if (!f) throw Error(MLXQ_EINVAL, "cannot open " + path);
  std::ostringstream ss;
  ss << f.rdbuf();
  return ss.str();
}

int64_t as_int(const Json* j, const std::string& what) {
  if (!j || !std::holds_alternative<int64_t>(j->v)) throw Error(MLXQ_EINVAL, "safetensors: bad " + what);
  return std::get<int64_t>(j->v);
}

}  // namespace

HostMap read_safetensors(const std::string& path) {
  // The length and the JSON header are read first; each tensor's byte range is then read from the
  // file straight into its buffer, so a multi-GB snapshot needs its own size in host memory once.
  std::ifstream f(path, std::ios::binary | std::ios::ate);
  if (!f) throw Error(MLXQ_EINVAL, "cannot open " + path);
  const uint64_t size = (uint64_t)f.tellg();
  if (size < 8) throw Error(MLXQ_EINVAL, "safetensors: " + path + " is too short");
  f.seekg(0);
  uint8_t len[8];
  f.read((char*)len, 8);
  uint64_t n = 0;
  for (int k = 7; k >= 0; --k) n = (n << 8) | len[k];
  if (!f || n > size - 8) throw Error(MLXQ_EINVAL, "safetensors: header length past the end of " + path);
  std::string head((size_t)n, '\0');
  f.read(head.data(), (std::streamsize)n);
  if (!f) throw Error(MLXQ_EINVAL, "safetensors: cannot read the header of " + path);
  const Json header = parse_json(head);
  const auto* obj = std::get_if<JsonObject>(&header.v);
  if (!obj) throw Error(MLXQ_EINVAL, "safetensors: header is not an object");
  const uint64_t base = 8 + n;
  HostMap out;
  for (const auto& [name, desc] : *obj) {
    if (name == "__metadata__") continue;
    const Json* dt = desc.get("dtype");
    const Json* shape = desc.get("shape");
    const Json* offs = desc.get("data_offsets");
    const auto* dims = shape ? std::get_if<JsonArray>(&shape->v) : nullptr;
    const auto* o = offs ? std::get_if<JsonArray>(&offs->v) : nullptr;
    if (!dt || !std::holds_alternative<std::string>(dt->v) || !dims || !o || o->size() != 2)
      throw Error(MLXQ_EINVAL, "safetensors: malformed entry " + name);
    HostTensor t;
    t.dtype = dtype_from_name(std::get<std::string>(dt->v));
    uint64_t count = 1;
    for (const Json& d : *dims) {
      const int64_t v = as_int(&d, "shape of " + name);
      if (v < 0 || (v > 0 && count > (UINT64_MAX / 16) / (uint64_t)v))
        throw Error(MLXQ_EINVAL, "safetensors: bad shape of " + name);
      t.shape.push_back(v);
      count *= (uint64_t)v;
    }
    const int64_t b = as_int(&(*o)[0], "offset"), e = as_int(&(*o)[1], "offset");
    if (b < 0 || e < b || (uint64_t)e > size - base || (uint64_t)(e - b) != count * dtype_size(t.dtype))
      throw Error(MLXQ_EINVAL, "safetensors: data range of " + name + " does not match its shape");
    t.data.resize((size_t)(e - b));
    f.seekg((std::streamoff)(base + (uint64_t)b));
    f.read((char*)t.data.data(), (std::streamsize)t.data.size());
    if (!f) throw Error(MLXQ_EINVAL, "safetensors: cannot read " + name + " from " + path);
    out.emplace(name, std::move(t));
  }
  return out;
}

void write_safetensors(const std::string& path, const HostMap& tensors) {
  Json header;
  header.v = JsonObject{};
  int64_t off = 0;
  for (const auto& [name, t] : tensors) {
    Json d;
    d.set("dtype", Json{std::string(dtype_name(t.dtype))});
    JsonArray shape;
    int64_t count = 1;
    for (int64_t s : t.shape) {
      shape.push_back(Json{s});
      count *= s;
    }
    if ((size_t)count * dtype_size(t.dtype) != t.data.size())
      throw Error(MLXQ_EINVAL, "safetensors: " + name + " holds the wrong number of bytes");
    d.set("shape", Json{shape});
    d.set("data_offsets", Json{JsonArray{Json{off}, Json{off + (int64_t)t.data.size()}}});
    header.set(name, d);
    off += (int64_t)t.data.size();
  }
  std::string h;
  dump_json(header, h, 0, 0);
  while ((8 + h.size()) % 8) h += ' ';  // data starts 8-byte aligned
  const auto parent = std::filesystem::path(path).parent_path();
  if (!parent.empty()) std::filesystem::create_directories(parent);
  std::ofstream f(path, std::ios::binary);
  if (!f) throw Error(MLXQ_EINVAL, "cannot write " + path);
  uint8_t len[8];
  for (int k = 0; k < 8; ++k) len[k] = (uint8_t)((uint64_t)h.size() >> (8 * k));
  f.write((const char*)len, 8);
  f.write(h.data(), (std::streamsize)h.size());
  for (const auto& kv : tensors) f.write((const char*)kv.second.data.data(), (std::streamsize)kv.second.data.size());
  if (!f) throw Error(MLXQ_EINVAL, "short write to " + path);
}

Weights load_dir_map(const std::string& dir) {
  std::vector<std::string> files;
  for (const auto& e : std::filesystem::directory_iterator(dir))
    if (e.is_regular_file() && e.path().extension() == ".safetensors") files.push_back(e.path().string());
  if (files.empty()) throw Error(MLXQ_EINVAL, "no *.safetensors under " + dir);
  std::sort(files.begin(), files.end());
  Weights out;
  for (const auto& f : files)
    for (auto& [name, t] : read_safetensors(f)) out[name] = Array::from_host(t.data.data(), t.shape, t.dtype);
  return out;
}

void save_map(const std::string& path, const Weights& map) {
  HostMap host;
  for (const auto& [name, a] : map) {
    HostTensor t;
    t.dtype = a.dtype();
    t.shape = a.shape();
    t.data.resize(a.nbytes());
    a.to_host(t.data.data());
    host.emplace(name, std::move(t));
  }
  write_safetensors(path, host);
}

void write_quantized_config(const std::string& src_dir, const std::string& dst_dir, int bits,
                            int group_size) {
  const auto src = std::filesystem::path(src_dir) / "config.json";
  Json cfg;
  cfg.v = JsonObject{};
  if (std::filesystem::exists(src)) cfg = parse_json(read_file(src.string()));
  if (!std::holds_alternative<JsonObject>(cfg.v)) throw Error(MLXQ_EINVAL, "config.json is not an object");
  Json q;
  q.set("bits", Json{(int64_t)bits});
  q.set("group_size", Json{(int64_t)group_size});
  cfg.set("quantization", q);
  std::string text;
  dump_json(cfg, text, 2, 0);
  std::filesystem::create_directories(dst_dir);
  std::ofstream f((std::filesystem::path(dst_dir) / "config.json").string());
  if (!f) throw Error(MLXQ_EINVAL, "cannot write config.json under " + dst_dir);
  f << text;
}

}  // namespace mlxq
