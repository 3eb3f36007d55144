// xrmm_execute: the job-JSON runner of xrGPU's extended operators
// (kernels/_shared/extended/tests/execute.cpp:14-35) over libxrmm's C ABI, so
// the reference's harness (kernels/_shared/extended/complex_reference.py:
// 751-836, which starts a runner per job as a subprocess) can drive libxrmm.
//
//   xrmm_execute JOB.json
//
// JOB: {"operation", "inputs": [tensor | null], "attrs", "args",
//       "outputs": [requested tensor descriptions], "plan_only", "profiling",
//       "timeout_ns", "memory_limit_bytes", "package", "repeat",
//       "output_directory"}
// tensor: {"name", "dtype", "storage_dtype"?, "shape", "layout"?,
//          "file" (raw little-endian bytes, relative to the job) |
//          "values" | "data" (nested literal arrays)}
// stdout (one line): {"planned_outputs": [...], "outputs": [... + "file"],
//                     "info": {...}}; outputs go to output<i>.bin in
// output_directory. Failures print {"error", "physical_qualification": false}
// on stderr and exit 1. Attribute values: booleans and integers become
// integer attributes, other numbers floats, strings strings; the operators
// here take no array or tensor attributes, so those are rejected by name.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <iostream>
#include <memory>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/xrmm.h"

namespace fs = std::filesystem;

namespace {

// ---------------------------------------------------------------------------
// a small JSON value and parser (objects keep their key order)

struct Json {
  enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
  bool b = false;
  std::string text;  // number literal or string value
  std::vector<Json> items;
  std::vector<std::pair<std::string, Json>> fields;

  const Json* find(const std::string& k) const {
    for (const auto& f : fields)
      if (f.first == k) return &f.second;
    return nullptr;
  }
  const Json& at(const std::string& k) const {
    const Json* v = find(k);
    if (!v) throw std::invalid_argument("Missing JSON key: " + k);
    return *v;
  }
  bool integral() const { return kind == Number && text.find_first_of(".eE") == std::string::npos; }
  bool negative() const { return kind == Number && !text.empty() && text[0] == '-'; }
  double num() const { return std::stod(text); }
  int64_t i64() const { return std::stoll(text); }
  uint64_t u64() const { return std::stoull(text); }
  std::string str() const {
    if (kind != String) throw std::invalid_argument("JSON string expected");
    return text;
  }
};

struct Parser {
  const std::string& s;
  size_t p = 0;
  // Nesting depth of the value being parsed. value() recurses per level, so
  // unbounded nesting in an untrusted file would overflow the stack; job
  // files nest four levels deep.
  int depth = 0;
  static constexpr int kMaxDepth = 64;
  struct Nest {
    Parser& q;
    explicit Nest(Parser& p_) : q(p_) {
      if (++q.depth > kMaxDepth) q.bad("nesting too deep");
    }
    ~Nest() { --q.depth; }
  };

  [[noreturn]] void bad(const char* what) const {
    throw std::invalid_argument(std::string("Invalid invocation JSON: ") + what + " at offset " + std::to_string(p));
  }
  void ws() {
    while (p < s.size() && (s[p] == ' ' || s[p] == '\n' || s[p] == '\r' || s[p] == '\t')) ++p;
  }
  bool lit(const char* w) {
    const size_t n = std::strlen(w);
    if (s.compare(p, n, w) == 0) {
      p += n;
      return true;
    }
    return false;
  }
  static void utf8(std::string& out, uint32_t c) {
    if (c < 0x80) {
      out += char(c);
    } else if (c < 0x800) {
      out += char(0xC0 | (c >> 6));
      out += char(0x80 | (c & 0x3F));
    } else if (c < 0x10000) {
      out += char(0xE0 | (c >> 12));
      out += char(0x80 | ((c >> 6) & 0x3F));
      out += char(0x80 | (c & 0x3F));
    } else {
      out += char(0xF0 | (c >> 18));
      out += char(0x80 | ((c >> 12) & 0x3F));
      out += char(0x80 | ((c >> 6) & 0x3F));
      out += char(0x80 | (c & 0x3F));
    }
  }
  uint32_t hex4() {
    if (p + 4 > s.size()) bad("short \\u escape");
    const uint32_t v = uint32_t(std::stoul(s.substr(p, 4), nullptr, 16));
    p += 4;
    return v;
  }
  std::string string() {
    if (s[p] != '"') bad("string expected");
    ++p;
    std::string out;
    while (true) {
      if (p >= s.size()) bad("unterminated string");
      const char c = s[p++];
      if (c == '"') break;
      if (c != '\\') {
        out += c;
        continue;
      }
      if (p >= s.size()) bad("bad escape");
      const char e = s[p++];
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
          uint32_t c1 = hex4();
          if (c1 >= 0xD800 && c1 < 0xDC00 && lit("\\u")) c1 = 0x10000 + ((c1 - 0xD800) << 10) + (hex4() - 0xDC00);
          utf8(out, c1);
          break;
        }
        default: bad("bad escape");
      }
    }
    return out;
  }
  Json value() {
    ws();
    if (p >= s.size()) bad("value expected");
    Json v;
    const char c = s[p];
    if (c == '{') {
      const Nest nest(*this);
      v.kind = Json::Object;
      ++p;
      ws();
      if (s[p] == '}') {
        ++p;
        return v;
      }
      while (true) {
        ws();
        std::string k = string();
        ws();
        if (s[p++] != ':') bad("':' expected");
        v.fields.emplace_back(std::move(k), value());
        ws();
        if (s[p] == ',') {
          ++p;
          continue;
        }
        if (s[p++] != '}') bad("'}' expected");
        return v;
      }
    }
    if (c == '[') {
      const Nest nest(*this);
      v.kind = Json::Array;
      ++p;
      ws();
      if (s[p] == ']') {
        ++p;
        return v;
      }
      while (true) {
        v.items.push_back(value());
        ws();
        if (s[p] == ',') {
          ++p;
          continue;
        }
        if (s[p++] != ']') bad("']' expected");
        return v;
      }
    }
    if (c == '"') {
      v.kind = Json::String;
      v.text = string();
      return v;
    }
    if (lit("true")) {
      v.kind = Json::Bool;
      v.b = true;
      return v;
    }
    if (lit("false")) {
      v.kind = Json::Bool;
      return v;
    }
    if (lit("null")) return v;
    const size_t q = p;
    if (s[p] == '-') ++p;
    while (p < s.size() && (std::isdigit(static_cast<unsigned char>(s[p])) || s[p] == '.' || s[p] == 'e' ||
                            s[p] == 'E' || s[p] == '+' || s[p] == '-'))
      ++p;
    if (q == p) bad("unexpected character");
    v.kind = Json::Number;
    v.text = s.substr(q, p - q);
    return v;
  }
};

Json parse(const std::string& text) {
  Parser ps{text};
  Json v = ps.value();
  ps.ws();
  if (ps.p != text.size()) ps.bad("trailing characters");
  return v;
}

std::string quote(const std::string& s) {
  std::string o = "\"";
  for (const unsigned char c : s) {
    if (c == '"' || c == '\\') {
      o += '\\';
      o += char(c);
    } else if (c < 0x20) {
      char buf[8];
      std::snprintf(buf, sizeof buf, "\\u%04x", c);
      o += buf;
    } else {
      o += char(c);
    }
  }
  return o + "\"";
}

// ---------------------------------------------------------------------------
// tensors and attributes

const char* kNames[] = {"float32", "float16", "int32", "uint32", "int16", "int8", "uint8", "int64", "bool", "unspecified"};

int32_t parse_dtype(const std::string& n) {
  for (int32_t i = 0; i <= XRMM_UNSPECIFIED; ++i)
    if (n == kNames[i]) return i;
  throw std::invalid_argument("Unsupported dtype: " + n);
}

uint32_t dtype_bytes(int32_t d) {
  switch (d) {
    case XRMM_F32: case XRMM_I32: case XRMM_U32: return 4;
    case XRMM_F16: case XRMM_I16: return 2;
    case XRMM_I8: case XRMM_U8: case XRMM_BOOL: return 1;
    case XRMM_I64: return 8;
    default: throw std::invalid_argument("Unsupported dtype");
  }
}

// IEEE binary16 bits of x, one rounding to nearest even (the reference's
// half_host::double_to_half): overflow to infinity, gradual underflow.
uint16_t to_half(double x) {
  uint64_t b;
  std::memcpy(&b, &x, 8);
  const uint16_t sign = uint16_t((b >> 48) & 0x8000);
  const int exp = int((b >> 52) & 0x7FF);
  const uint64_t mant = b & ((uint64_t(1) << 52) - 1);
  if (exp == 0x7FF) return uint16_t(sign | 0x7C00 | (mant ? 0x200 : 0));
  if (exp == 0) return sign;  // double subnormals are far below half's range
  const int e = exp - 1023;
  if (e > 15) return uint16_t(sign | 0x7C00);
  const uint64_t full = (uint64_t(1) << 52) | mant;
  // normal half: 10 kept mantissa bits; subnormal half: units of 2^-24
  const int shift = e >= -14 ? 42 : 52 - (e + 24);
  if (shift > 62) return sign;
  uint64_t m = (e >= -14 ? mant : full) >> shift;
  const uint64_t rem = (e >= -14 ? mant : full) & ((uint64_t(1) << shift) - 1), half = uint64_t(1) << (shift - 1);
  if (e >= -14) m |= uint64_t(e + 15) << 10;
  if (rem > half || (rem == half && (m & 1))) ++m;  // a carry moves into the exponent, up to infinity
  return uint16_t(sign | m);
}

// Literal numbers (execute.cpp:14): strings must parse whole, booleans are 0/1.
double number(const Json& j) {
  if (j.kind == Json::String) {
    size_t used = 0;
    const double v = std::stod(j.text, &used);
    if (used != j.text.size()) throw std::invalid_argument("Invalid numeric literal");
    return v;
  }
  if (j.kind == Json::Bool) return j.b ? 1 : 0;
  if (j.kind != Json::Number) throw std::invalid_argument("Invalid numeric literal");
  return j.num();
}

void flatten(const Json& a, std::vector<const Json*>& out) {
  if (a.kind == Json::Array)
    for (const auto& x : a.items) flatten(x, out);
  else
    out.push_back(&a);
}

struct OwnedTensor {
  std::string name;
  int32_t dtype = XRMM_UNSPECIFIED, storage = XRMM_UNSPECIFIED;
  std::vector<int64_t> shape;
  std::vector<uint8_t> data;

  xrmm_tensor view() const {
    xrmm_tensor t{};
    t.name = name.c_str();
    t.dtype = dtype;
    t.storage_dtype = storage;
    t.rank = int32_t(shape.size());
    for (size_t i = 0; i < shape.size() && i < XRMM_MAX_RANK; ++i) t.shape[i] = shape[i];
    t.data = data.empty() ? nullptr : data.data();
    t.nbytes = data.size();
    return t;
  }
};

OwnedTensor tensor(const Json& j, const fs::path& base, bool payload, const std::string& fallback = "") {
  OwnedTensor t;
  const Json* nm = j.find("name");
  t.name = nm ? nm->str() : fallback;
  t.dtype = parse_dtype(j.at("dtype").str());
  if (const Json* sd = j.find("storage_dtype")) t.storage = parse_dtype(sd->str());
  for (const auto& d : j.at("shape").items) t.shape.push_back(d.i64());
  if (t.shape.size() > XRMM_MAX_RANK) throw std::invalid_argument("Rank outside the supported range: " + t.name);
  if (const Json* lay = j.find("layout"))
    if (lay->str() != "contiguous") throw std::invalid_argument("Only contiguous layouts are supported: " + t.name);
  if (!payload) return t;
  const int32_t storage = t.storage == XRMM_UNSPECIFIED ? t.dtype : t.storage;
  uint64_t count = 1;
  for (const int64_t d : t.shape) {
    if (d < 0) throw std::invalid_argument("Negative dimension: " + t.name);
    count *= uint64_t(d);
  }
  const uint32_t bytes = dtype_bytes(storage);
  if (const Json* f = j.find("file")) {
    fs::path path = f->str();
    if (path.is_relative()) path = base / path;
    std::ifstream in(path, std::ios::binary | std::ios::ate);
    if (!in || in.tellg() != std::streamoff(count * bytes))
      throw std::invalid_argument("Tensor file byte count mismatch: " + path.string());
    t.data.resize(count * bytes);
    in.seekg(0);
    if (!t.data.empty()) in.read(reinterpret_cast<char*>(t.data.data()), std::streamsize(t.data.size()));
    if (!in) throw std::invalid_argument("Tensor file read failed: " + path.string());
    return t;
  }
  std::vector<const Json*> values;
  if (const Json* v = j.find("values"))
    flatten(*v, values);
  else if (const Json* d = j.find("data"))
    flatten(*d, values);
  if (values.size() != count) throw std::invalid_argument("Literal tensor value count mismatch");
  t.data.resize(count * bytes);
  for (size_t i = 0; i < values.size(); ++i) {
    const Json& v = *values[i];
    uint64_t bits = 0;
    if (storage == XRMM_F32) {
      const float x = float(number(v));
      uint32_t b;
      std::memcpy(&b, &x, 4);
      bits = b;
    } else if (storage == XRMM_F16) {
      bits = to_half(number(v));
    } else if (storage == XRMM_BOOL) {
      bits = number(v) != 0;
    } else if (v.integral() && !v.negative()) {
      bits = v.u64();
    } else if (v.integral()) {
      bits = uint64_t(v.i64());
    } else {
      bits = uint64_t(int64_t(number(v)));
    }
    std::memcpy(t.data.data() + i * bytes, &bits, bytes);
  }
  return t;
}

struct OwnedAttrs {
  std::vector<std::string> keys, strs;
  std::vector<xrmm_attr> list;
};

void attributes(const Json* j, OwnedAttrs& a) {
  if (!j || j->kind == Json::Null) return;
  if (j->kind != Json::Object) throw std::invalid_argument("Attributes/args require objects");
  a.keys.reserve(j->fields.size());
  a.strs.reserve(j->fields.size());
  for (const auto& f : j->fields) {
    const Json& v = f.second;
    xrmm_attr x{};
    a.keys.push_back(f.first);
    if (v.kind == Json::Bool) {
      x.kind = XRMM_ATTR_INT;
      x.i = v.b ? 1 : 0;
    } else if (v.kind == Json::Number && v.integral()) {
      x.kind = XRMM_ATTR_INT;
      x.i = v.i64();
    } else if (v.kind == Json::Number) {
      x.kind = XRMM_ATTR_FLOAT;
      x.f = v.num();
    } else if (v.kind == Json::String) {
      x.kind = XRMM_ATTR_STRING;
      a.strs.push_back(v.text);
    } else {
      throw std::invalid_argument("Unsupported native attribute encoding: " + f.first);
    }
    a.list.push_back(x);
  }
  size_t si = 0;
  for (size_t i = 0; i < a.list.size(); ++i) {
    a.list[i].key = a.keys[i].c_str();
    if (a.list[i].kind == XRMM_ATTR_STRING) a.list[i].s = a.strs[si++].c_str();
  }
}

std::string describe(const xrmm_tensor_desc& d, const std::string& file = "") {
  std::ostringstream o;
  o << "{\"name\":" << quote(d.name) << ",\"dtype\":" << quote(kNames[d.dtype])
    << ",\"storage_dtype\":" << quote(kNames[d.storage_dtype]) << ",\"shape\":[";
  for (int32_t i = 0; i < d.rank; ++i) o << (i ? "," : "") << d.shape[i];
  o << "],\"layout\":\"contiguous\"";
  if (!file.empty()) o << ",\"file\":" << quote(file);
  return o.str() + "}";
}

void check(int rc) {
  if (rc == XRMM_OK) return;
  const std::string why = xrmm_last_error();
  if (rc == XRMM_EINVAL) throw std::invalid_argument(why);
  throw std::runtime_error(why);
}

int run_job(const char* path) {
  const fs::path job = fs::absolute(path);
  std::ifstream in(job);
  if (!in) throw std::invalid_argument("Cannot read invocation JSON");
  std::stringstream buf;
  buf << in.rdbuf();
  const Json j = parse(buf.str());
  const fs::path base = job.parent_path();

  const std::string operation = j.at("operation").str();
  std::vector<OwnedTensor> inputs, requested;
  if (const Json* ins = j.find("inputs"))
    for (const auto& t : ins->items)
      if (t.kind != Json::Null) inputs.push_back(tensor(t, base, true));
  if (const Json* outs = j.find("outputs"))
    for (const auto& t : outs->items) requested.push_back(tensor(t, base, false));
  OwnedAttrs attrs, args;
  attributes(j.find("attrs"), attrs);
  attributes(j.find("args"), args);
  std::vector<xrmm_tensor> in_views, req_views;
  for (const auto& t : inputs) in_views.push_back(t.view());
  for (const auto& t : requested) req_views.push_back(t.view());
  xrmm_request r{};
  r.operation = operation.c_str();
  r.inputs = in_views.data();
  r.n_inputs = int32_t(in_views.size());
  r.attrs = attrs.list.data();
  r.n_attrs = int32_t(attrs.list.size());
  r.args = args.list.data();
  r.n_args = int32_t(args.list.size());
  r.requested_outputs = req_views.data();
  r.n_requested_outputs = int32_t(req_views.size());

  int32_t n = 0;
  check(xrmm_plan(&r, nullptr, 0, &n));
  std::vector<xrmm_tensor_desc> planned(size_t(n > 0 ? n : 0));
  check(xrmm_plan(&r, planned.data(), n, &n));
  std::string planned_json = "[";
  for (int32_t i = 0; i < n; ++i) planned_json += (i ? "," : "") + describe(planned[i]);
  planned_json += "]";

  const Json* po = j.find("plan_only");
  if (po && (po->kind == Json::Bool ? po->b : po->kind == Json::Number && po->num() != 0)) {
    std::cout << "{\"planned_outputs\":" << planned_json << ",\"info\":{\"backend\":\"host_shape_plan\",\"test_only\":true,"
              << "\"physical_qualification\":false,\"operation\":" << quote(operation)
              << ",\"extended\":true,\"shader\":\"xrmm\"},\"outputs\":" << planned_json << "}\n";
    return 0;
  }

  xrmm_options o;
  xrmm_default_options(&o);
  if (const Json* v = j.find("profiling")) o.profiling = v->kind == Json::Bool ? v->b : int32_t(number(*v));
  if (const Json* v = j.find("timeout_ns")) o.timeout_ns = v->u64();
  if (const Json* v = j.find("memory_limit_bytes")) o.memory_limit_bytes = v->u64();
  (void)j.at("package").str();  // required by the wire format; the kernels are linked into libxrmm
  const Json* rep = j.find("repeat");
  const int64_t repeat = rep ? rep->i64() : 1;
  if (repeat < 1 || repeat > 1000) throw std::invalid_argument("Invalid repeat count");
  fs::path dir = j.at("output_directory").str();
  if (dir.is_relative()) dir = base / dir;

  xrmm_op* raw = nullptr;
  check(xrmm_prepare(&r, &o, &raw));
  std::unique_ptr<xrmm_op, void (*)(xrmm_op*)> op(raw, xrmm_destroy);
  for (int64_t i = 0; i < repeat; ++i) check(xrmm_run(op.get()));
  check(xrmm_output_descs(op.get(), planned.data(), n, &n));
  std::vector<std::vector<uint8_t>> outs(size_t(n > 0 ? n : 0));
  std::vector<void*> ptrs;
  std::vector<uint64_t> sizes;
  for (int32_t i = 0; i < n; ++i) {
    outs[i].resize(planned[i].nbytes);
    ptrs.push_back(outs[i].empty() ? nullptr : outs[i].data());
    sizes.push_back(planned[i].nbytes);
  }
  check(xrmm_read_outputs(op.get(), ptrs.data(), sizes.data(), n));
  fs::create_directories(dir);
  std::string out_json = "[";
  for (int32_t i = 0; i < n; ++i) {
    const fs::path file = dir / ("output" + std::to_string(i) + ".bin");
    std::ofstream f(file, std::ios::binary);
    if (!outs[i].empty()) f.write(reinterpret_cast<const char*>(outs[i].data()), std::streamsize(outs[i].size()));
    if (!f) throw std::runtime_error("Output file write failed");
    out_json += (i ? "," : "") + describe(planned[i], file.string());
  }
  out_json += "]";
  const std::string info = xrmm_info(op.get());
  check(xrmm_close(op.get()));
  std::cout << "{\"planned_outputs\":" << planned_json << ",\"outputs\":" << out_json << ",\"info\":" << info << "}\n";
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  try {
    if (argc != 2) throw std::invalid_argument("Usage: xrmm_execute JOB.json");
    return run_job(argv[1]);
  } catch (const std::exception& e) {
    std::cerr << "{\"error\":" << quote(e.what()) << ",\"physical_qualification\":false}\n";
    return 1;
  }
}
