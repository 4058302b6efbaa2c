// loader.cpp -- model weight files in the two formats the reference reads
// (internal/embeddings/weights/loader.go): a raw little-endian float32 stream
// in a fixed tensor order (LoadFromRawBinary, loader.go:29-90) and SafeTensors
// with HuggingFace BERT names (LoadFromSafeTensors, loader.go:155-237).
//
// Both walk the same ordered list of the model's tensors: the shapes are the
// ones NewBertModel allocates (bert.go:191-193, 279-280, 396-397, 542-547,
// 742-743, 776-777, 807-808), the order and names are the loader's.  Each
// tensor is handed to fl_model_set_weight, so the device-side conversion and
// repacking is the same as for weights uploaded one by one.
//
// Reference behaviour kept: the raw stream must hold at least every tensor
// (trailing bytes are ignored); SafeTensors tensors are matched by name, must
// have the element count of the model tensor, must be F32, and 2-D ".weight"
// tensors outside the embeddings and LayerNorms are HF [out, in] matrices
// transposed to the model's [in, out].  Deliberate differences: errors are
// status codes with the message in fl_last_error(); a bias-free model (Nomic)
// rejects a file whose biases are not all zero instead of ignoring them; the
// position table of a RoPE model is read and discarded (bert.go:222 never
// reads it).
#include <cerrno>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "context.hpp"

namespace {

using fl::fail;

struct Slot {
  std::string hf;    // SafeTensors name (loader.go:199-236)
  std::string name;  // fl_model_set_weight name
  int64_t rows, cols;
  bool bias;         // a projection bias (must be zero for bias-free models)
};

// Tensors in LoadFromRawBinary order (loader.go:40-88), which is also the
// order LoadFromSafeTensors visits them (loader.go:199-236).
std::vector<Slot> reference_order(const fl_model_config& c) {
  const int64_t H = c.hidden, I = c.intermediate;
  const int64_t Ni = c.activation == FL_ACT_SWIGLU ? 2 * I : I;  // bert.go:769-772
  std::vector<Slot> s;
  s.push_back({"embeddings.word_embeddings.weight", "word_emb", c.vocab_size, H, false});
  s.push_back({"embeddings.position_embeddings.weight", "pos_emb", c.max_pos, H, false});
  s.push_back({"embeddings.token_type_embeddings.weight", "type_emb", 2, H, false});
  s.push_back({"embeddings.LayerNorm.weight", "emb_ln_g", 1, H, false});
  s.push_back({"embeddings.LayerNorm.bias", "emb_ln_b", 1, H, false});
  for (int l = 0; l < c.layers; ++l) {
    const std::string p = "encoder.layer." + std::to_string(l), n = "." + std::to_string(l);
    const char* qkv[3][2] = {{"query", "q"}, {"key", "k"}, {"value", "v"}};
    for (auto& f : qkv) {
      s.push_back({p + ".attention.self." + f[0] + ".weight", std::string(f[1]) + "_w" + n, H, H, false});
      s.push_back({p + ".attention.self." + f[0] + ".bias", std::string(f[1]) + "_b" + n, 1, H, true});
    }
    s.push_back({p + ".attention.output.dense.weight", "o_w" + n, H, H, false});
    s.push_back({p + ".attention.output.dense.bias", "o_b" + n, 1, H, true});
    s.push_back({p + ".attention.output.LayerNorm.weight", "attn_ln_g" + n, 1, H, false});
    s.push_back({p + ".attention.output.LayerNorm.bias", "attn_ln_b" + n, 1, H, false});
    s.push_back({p + ".intermediate.dense.weight", "inter_w" + n, H, Ni, false});
    s.push_back({p + ".intermediate.dense.bias", "inter_b" + n, 1, Ni, true});
    s.push_back({p + ".output.dense.weight", "out_w" + n, I, H, false});
    s.push_back({p + ".output.dense.bias", "out_b" + n, 1, H, true});
    s.push_back({p + ".output.LayerNorm.weight", "out_ln_g" + n, 1, H, false});
    s.push_back({p + ".output.LayerNorm.bias", "out_ln_b" + n, 1, H, false});
  }
  s.push_back({"pooler.dense.weight", "pool_w", H, H, false});
  // The pooler keeps its bias in every model (bert.go:396-397).
  s.push_back({"pooler.dense.bias", "pool_b", 1, H, false});
  return s;
}

// Hands one tensor (reference [rows, cols] layout) to the model.
int store(fl_model* m, const fl_model_config& c, const Slot& s, const std::vector<float>& v) {
  if (s.bias && !c.has_bias) {
    for (float x : v)
      if (x != 0.f)
        return fail(FL_ERR_INVALID, "tensor " + s.hf + " is not zero but the model has no biases");
    return FL_OK;  // the model's bias buffers are zero already and never read
  }
  if (s.name == "pos_emb" && c.position == FL_POS_ROPE) return FL_OK;
  return fl_model_set_weight(m, s.name.c_str(), v.data(), (int64_t)v.size());
}

struct File {
  FILE* f = nullptr;
  ~File() {
    if (f) std::fclose(f);
  }
};

int open_file(const char* path, File& out, int64_t& size) {
  if (!path) return fail(FL_ERR_INVALID, "null path");
  out.f = std::fopen(path, "rb");
  if (!out.f) return fail(FL_ERR_IO, std::string("open ") + path + ": " + std::strerror(errno));
  if (std::fseek(out.f, 0, SEEK_END) != 0) return fail(FL_ERR_IO, std::string("seek ") + path);
  size = (int64_t)std::ftell(out.f);
  if (size < 0 || std::fseek(out.f, 0, SEEK_SET) != 0) return fail(FL_ERR_IO, std::string("seek ") + path);
  return FL_OK;
}

// ---- a JSON reader for the SafeTensors header -------------------------------
// The header is one object: name -> {"dtype": str, "shape": [int...],
// "data_offsets": [int, int]}, plus an optional "__metadata__" object of
// strings.  This reader accepts general JSON values and keeps what it needs.
struct Json {
  enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
  double num = 0;
  bool integral = false;
  int64_t inum = 0;
  std::string str;
  std::vector<Json> arr;
  std::map<std::string, Json> obj;
};

struct Parser {
  const char* p;
  const char* e;
  std::string err;

  void ws() {
    while (p < e && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
  }
  bool bad(const char* what) {
    if (err.empty()) err = what;
    return false;
  }
  bool lit(const char* s) {
    const size_t n = std::strlen(s);
    if ((size_t)(e - p) < n || std::memcmp(p, s, n) != 0) return bad("bad literal");
    p += n;
    return true;
  }
  bool string(std::string& out) {
    if (p >= e || *p != '"') return bad("expected string");
    ++p;
    while (p < e && *p != '"') {
      char ch = *p++;
      if (ch != '\\') {
        out.push_back(ch);
        continue;
      }
      if (p >= e) return bad("bad escape");
      ch = *p++;
      switch (ch) {
        case '"': case '\\': case '/': out.push_back(ch); break;
        case 'b': out.push_back('\b'); break;
        case 'f': out.push_back('\f'); break;
        case 'n': out.push_back('\n'); break;
        case 'r': out.push_back('\r'); break;
        case 't': out.push_back('\t'); break;
        case 'u': {
          if (e - p < 4) return bad("bad \\u escape");
          unsigned cp = 0;
          for (int i = 0; i < 4; ++i) {
            const char h = *p++;
            cp <<= 4;
            if (h >= '0' && h <= '9') cp |= (unsigned)(h - '0');
            else if (h >= 'a' && h <= 'f') cp |= (unsigned)(h - 'a' + 10);
            else if (h >= 'A' && h <= 'F') cp |= (unsigned)(h - 'A' + 10);
            else return bad("bad \\u escape");
          }
          // UTF-8 of the code unit (surrogate pairs are kept as two units;
          // tensor names are ASCII in practice).
          if (cp < 0x80) out.push_back((char)cp);
          else if (cp < 0x800) { out.push_back((char)(0xC0 | (cp >> 6))); out.push_back((char)(0x80 | (cp & 63))); }
          else { out.push_back((char)(0xE0 | (cp >> 12))); out.push_back((char)(0x80 | ((cp >> 6) & 63))); out.push_back((char)(0x80 | (cp & 63))); }
          break;
        }
        default: return bad("bad escape");
      }
    }
    if (p >= e) return bad("unterminated string");
    ++p;
    return true;
  }
  bool number(Json& j) {
    const char* s = p;
    if (p < e && *p == '-') ++p;
    bool frac = false;
    while (p < e && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' || *p == '+' || *p == '-')) {
      if (*p == '.' || *p == 'e' || *p == 'E') frac = true;
      ++p;
    }
    if (p == s) return bad("expected value");
    const std::string t(s, p);
    char* end = nullptr;
    j.kind = Json::NUM;
    j.num = std::strtod(t.c_str(), &end);
    if (!end || *end) return bad("bad number");
    if (!frac) {
      errno = 0;
      j.inum = std::strtoll(t.c_str(), &end, 10);
      j.integral = errno == 0 && end && !*end;
    }
    return true;
  }
  bool value(Json& j, int depth) {
    if (depth > 64) return bad("nesting too deep");
    ws();
    if (p >= e) return bad("unexpected end");
    switch (*p) {
      case '{': {
        ++p;
        j.kind = Json::OBJ;
        ws();
        if (p < e && *p == '}') { ++p; return true; }
        for (;;) {
          ws();
          std::string k;
          if (!string(k)) return false;
          ws();
          if (p >= e || *p != ':') return bad("expected ':'");
          ++p;
          Json v;
          if (!value(v, depth + 1)) return false;
          j.obj[k] = std::move(v);
          ws();
          if (p < e && *p == ',') { ++p; continue; }
          if (p < e && *p == '}') { ++p; return true; }
          return bad("expected ',' or '}'");
        }
      }
      case '[': {
        ++p;
        j.kind = Json::ARR;
        ws();
        if (p < e && *p == ']') { ++p; return true; }
        for (;;) {
          Json v;
          if (!value(v, depth + 1)) return false;
          j.arr.push_back(std::move(v));
          ws();
          if (p < e && *p == ',') { ++p; continue; }
          if (p < e && *p == ']') { ++p; return true; }
          return bad("expected ',' or ']'");
        }
      }
      case '"': j.kind = Json::STR; return string(j.str);
      case 't': j.kind = Json::BOOL; return lit("true");
      case 'f': j.kind = Json::BOOL; return lit("false");
      case 'n': j.kind = Json::NUL; return lit("null");
      default: return number(j);
    }
  }
};

struct TensorInfo {
  std::string dtype;
  std::vector<int64_t> shape;
  int64_t begin = 0, end = 0;
};

int header_entry(const std::string& name, const Json& j, TensorInfo& t) {
  auto bad = [&](const char* what) {
    return fail(FL_ERR_IO, "safetensors header: tensor " + name + ": " + what);
  };
  if (j.kind != Json::OBJ) return bad("not an object");
  auto d = j.obj.find("dtype"), s = j.obj.find("shape"), o = j.obj.find("data_offsets");
  if (d == j.obj.end() || d->second.kind != Json::STR) return bad("missing dtype");
  if (s == j.obj.end() || s->second.kind != Json::ARR) return bad("missing shape");
  if (o == j.obj.end() || o->second.kind != Json::ARR || o->second.arr.size() != 2) return bad("missing data_offsets");
  t.dtype = d->second.str;
  for (const Json& x : s->second.arr) {
    if (x.kind != Json::NUM || !x.integral || x.inum < 0) return bad("bad shape");
    t.shape.push_back(x.inum);
  }
  const Json &b = o->second.arr[0], &e = o->second.arr[1];
  if (b.kind != Json::NUM || !b.integral || e.kind != Json::NUM || !e.integral || b.inum < 0 || e.inum < b.inum)
    return bad("bad data_offsets");
  t.begin = b.inum;
  t.end = e.inum;
  return FL_OK;
}

bool ends_with(const std::string& s, const char* suf) {
  const size_t n = std::strlen(suf);
  return s.size() >= n && s.compare(s.size() - n, n, suf) == 0;
}

}  // namespace

int fl_model_load_raw(fl_model* m, const char* path) {
  if (!m) return fail(FL_ERR_INVALID, "null model");
  const fl_model_config& c = *fl::model_config(m);
  File f;
  int64_t size = 0;
  if (int st = open_file(path, f, size)) return st;
  std::vector<float> v;
  for (const Slot& s : reference_order(c)) {
    v.resize((size_t)(s.rows * s.cols));
    // loader.go:95-110: binary.Read of rows*cols little-endian float32 (the
    // host is little-endian); a short read is an error.
    if (std::fread(v.data(), 4, v.size(), f.f) != v.size())
      return fail(FL_ERR_IO, "raw weights " + std::string(path) + ": unexpected end of file in " + s.hf);
    if (int st = store(m, c, s, v)) return st;
  }
  return FL_OK;
}

int fl_model_load_safetensors(fl_model* m, const char* path) {
  if (!m) return fail(FL_ERR_INVALID, "null model");
  const fl_model_config& c = *fl::model_config(m);
  File f;
  int64_t size = 0;
  if (int st = open_file(path, f, size)) return st;
  // loader.go:163-180: u64 little-endian header length, then the JSON header
  // (at most 100 MB).
  uint64_t hlen = 0;
  if (size < 8 || std::fread(&hlen, 8, 1, f.f) != 1)
    return fail(FL_ERR_IO, "safetensors: failed to read header size");
  if (hlen > 100ull * 1024 * 1024) return fail(FL_ERR_IO, "safetensors: header size too large: " + std::to_string(hlen));
  if ((int64_t)hlen > size - 8) return fail(FL_ERR_IO, "safetensors: header runs past the end of the file");
  std::string hdr((size_t)hlen, '\0');
  if (hlen && std::fread(&hdr[0], 1, hlen, f.f) != hlen) return fail(FL_ERR_IO, "safetensors: failed to read header");
  Parser ps{hdr.data(), hdr.data() + hdr.size(), {}};
  Json root;
  if (!ps.value(root, 0) || root.kind != Json::OBJ)
    return fail(FL_ERR_IO, "safetensors: failed to parse header JSON: " + (ps.err.empty() ? "not an object" : ps.err));
  const int64_t data_start = 8 + (int64_t)hlen;  // offsets are relative to the body

  std::vector<float> v, t;
  for (const Slot& s : reference_order(c)) {
    auto it = root.obj.find(s.hf);
    if (it == root.obj.end()) return fail(FL_ERR_INVALID, "tensor \"" + s.hf + "\" not found in SafeTensors file");
    TensorInfo ti;
    if (int st = header_entry(s.hf, it->second, ti)) return st;
    const int64_t want = s.rows * s.cols;
    int64_t have = 1;
    bool overflow = false;
    std::string shp;
    for (int64_t d : ti.shape) {
      overflow |= __builtin_mul_overflow(have, d, &have);
      shp += (shp.empty() ? "" : " ") + std::to_string(d);
    }
    if (overflow)
      return fail(FL_ERR_IO, "tensor \"" + s.hf + "\": shape [" + shp + "] overflows 64 bits");
    if (have != want)
      return fail(FL_ERR_INVALID, "tensor \"" + s.hf + "\" size mismatch: expected " + std::to_string(want) +
                                      ", got " + std::to_string(have) + " (shape [" + shp + "])");
    const int64_t len = ti.end - ti.begin;
    if (ti.dtype == "F16" && len == want * 2)
      return fail(FL_ERR_UNSUPPORTED, "tensor \"" + s.hf + "\" is F16, only F32 supported currently");
    if (len != want * 4)
      return fail(FL_ERR_INVALID, "tensor \"" + s.hf + "\" byte size mismatch: expected " + std::to_string(want * 4) +
                                      ", got " + std::to_string(len));
    if (ti.dtype != "F32") return fail(FL_ERR_UNSUPPORTED, "tensor \"" + s.hf + "\" has dtype " + ti.dtype + ", only F32 supported");
    // ti.end >= 0 and data_start <= size (header checks), so this cannot overflow.
    if (ti.end > size - data_start)
      return fail(FL_ERR_IO, "tensor \"" + s.hf + "\": data runs past the end of the file");
    v.resize((size_t)want);
    if (std::fseek(f.f, (long)(data_start + ti.begin), SEEK_SET) != 0 || std::fread(v.data(), 4, v.size(), f.f) != v.size())
      return fail(FL_ERR_IO, "failed to read data for \"" + s.hf + "\"");
    // loader.go:209-229: 2-D ".weight" tensors outside the embeddings and
    // LayerNorms are [out, in] and become [in, out].
    const bool linear = ends_with(s.hf, ".weight") && ti.shape.size() == 2 &&
                        s.hf.find("embeddings") == std::string::npos && s.hf.find("LayerNorm") == std::string::npos;
    if (linear) {
      const int64_t out_rows = ti.shape[0], in_cols = ti.shape[1];
      if (out_rows != s.cols || in_cols != s.rows)
        return fail(FL_ERR_INVALID, "tensor \"" + s.hf + "\" shape mismatch for transpose: header=[" + shp +
                                        "], expected (" + std::to_string(s.rows) + ", " + std::to_string(s.cols) + ")");
      t.resize(v.size());
      for (int64_t i = 0; i < out_rows; ++i)
        for (int64_t j = 0; j < in_cols; ++j) t[(size_t)(j * out_rows + i)] = v[(size_t)(i * in_cols + j)];
      v.swap(t);
    }
    if (int st = store(m, c, s, v)) return st;
  }
  return FL_OK;
}
