// arena.cpp -- weight files into a decoder.
//
// The reference loads decoder weights from a baked safetensors "arena"
// (rust/npu-weights/src/arena.rs:14-99: bf16 linears and f32 vectors, header
// metadata `arch` and `format_version` = 1, lib.rs:11), whose names and
// layouts its arch modules fix (arch/opt.rs:1-123: `embed_tokens`,
// `L{i}/q.weight` stored transposed [in, out], `L{i}/q.bias`, `L{i}/ln_self.*`,
// `L{i}/ln_ffn.*`, ...), and bakes that arena from Hugging Face checkpoints
// (scripts/convert_opt125m.py, arch/opt.rs:119-123).  xe_decoder_load_safetensors
// reads either naming directly: the file is mapped, the JSON header parsed,
// every tensor converted to fp32 [out, in] and handed to xe_decoder_set_tensor,
// which quantises it to the decoder's weight type as for any fp32 upload.
// Everything here runs on the host, once per model load.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cctype>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <map>
#include <set>

#include "common.h"
#include "quant.h"

namespace xe {
namespace {

// ---------------------------------------------------------------------------
// JSON (the safetensors header: objects, arrays, strings, integers)
// ---------------------------------------------------------------------------
struct JVal {
  enum Type { NUL, NUM, STR, ARR, OBJ } t = NUL;
  double num = 0;
  std::string str;
  std::vector<JVal> arr;
  std::vector<std::pair<std::string, JVal>> obj;
  const JVal *get(const std::string &k) const {
    for (const auto &kv : obj)
      if (kv.first == k) return &kv.second;
    return nullptr;
  }
};

struct JParser {
  const char *p, *end;
  void ws() {
    while (p < end && std::isspace(static_cast<unsigned char>(*p))) p++;
  }
  [[noreturn]] void bad(const char *what) { fail(std::string("safetensors header: ") + what); }
  std::string string() {
    if (p >= end || *p != '"') bad("string expected");
    p++;
    std::string s;
    while (p < end && *p != '"') {
      if (*p == '\\') {
        p++;
        if (p >= end) bad("bad escape");
        switch (*p) {
          case 'n': s += '\n'; break;
          case 't': s += '\t'; break;
          case 'r': s += '\r'; break;
          case 'b': s += '\b'; break;
          case 'f': s += '\f'; break;
          case 'u': {  // keep ASCII code points; others become '?'
            if (end - p < 5) bad("bad \\u escape");
            const unsigned v = static_cast<unsigned>(std::strtoul(std::string(p + 1, p + 5).c_str(), nullptr, 16));
            s += v < 128 ? static_cast<char>(v) : '?';
            p += 4;
            break;
          }
          default: s += *p;
        }
        p++;
      } else {
        s += *p++;
      }
    }
    if (p >= end) bad("unterminated string");
    p++;
    return s;
  }
  JVal value(int depth = 0) {
    if (depth > 16) bad("nesting too deep");
    ws();
    if (p >= end) bad("unexpected end");
    JVal v;
    if (*p == '{') {
      v.t = JVal::OBJ;
      p++;
      ws();
      if (p < end && *p == '}') {
        p++;
        return v;
      }
      while (true) {
        ws();
        std::string k = string();
        ws();
        if (p >= end || *p != ':') bad("':' expected");
        p++;
        v.obj.emplace_back(std::move(k), value(depth + 1));
        ws();
        if (p < end && *p == ',') {
          p++;
          continue;
        }
        if (p < end && *p == '}') {
          p++;
          return v;
        }
        bad("',' or '}' expected");
      }
    }
    if (*p == '[') {
      v.t = JVal::ARR;
      p++;
      ws();
      if (p < end && *p == ']') {
        p++;
        return v;
      }
      while (true) {
        v.arr.push_back(value(depth + 1));
        ws();
        if (p < end && *p == ',') {
          p++;
          continue;
        }
        if (p < end && *p == ']') {
          p++;
          return v;
        }
        bad("',' or ']' expected");
      }
    }
    if (*p == '"') {
      v.t = JVal::STR;
      v.str = string();
      return v;
    }
    if (*p == '-' || std::isdigit(static_cast<unsigned char>(*p))) {
      char *e = nullptr;
      v.t = JVal::NUM;
      v.num = std::strtod(p, &e);
      if (e == p || e > end) bad("bad number");
      p = e;
      return v;
    }
    if (end - p >= 4 && std::strncmp(p, "null", 4) == 0) {
      p += 4;
      return v;
    }
    bad("unexpected character");
  }
};

// ---------------------------------------------------------------------------
// a mapped safetensors file
// ---------------------------------------------------------------------------
struct TensorRef {
  std::string dtype;  // F32 / BF16 / F16
  std::vector<int64_t> shape;
  const uint8_t *data = nullptr;
  size_t bytes = 0;
};

// A JSON number that must be a non-negative integer below 2^53 (exact in a
// double): shape entries and data offsets.
size_t json_index(const JVal &v, const std::string &what) {
  XE_REQUIRE(v.t == JVal::NUM && v.num >= 0.0 && v.num < 9007199254740992.0 && std::floor(v.num) == v.num,
             "safetensors header: " + what + " must be a non-negative integer");
  return static_cast<size_t>(v.num);
}

struct StFile {
  int fd = -1;
  void *map = nullptr;
  size_t size = 0;
  std::map<std::string, std::string> meta;
  std::map<std::string, TensorRef> tensors;
  explicit StFile(const char *path) {
    XE_REQUIRE(path, "null path");
    fd = ::open(path, O_RDONLY);
    XE_REQUIRE(fd >= 0, std::string("cannot open ") + path);
    struct stat st;
    XE_REQUIRE(::fstat(fd, &st) == 0, std::string("cannot stat ") + path);
    size = static_cast<size_t>(st.st_size);
    XE_REQUIRE(size >= 8, std::string(path) + ": not a safetensors file (too short)");
    map = ::mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
    XE_REQUIRE(map != MAP_FAILED, std::string("cannot map ") + path);
    const uint8_t *b = static_cast<const uint8_t *>(map);
    uint64_t hlen = 0;
    for (int i = 7; i >= 0; i--) hlen = hlen << 8 | b[i];  // little-endian u64
    XE_REQUIRE(hlen > 0 && hlen <= size - 8 && hlen < (uint64_t(100) << 20),
               std::string(path) + ": bad safetensors header length");
    // the header is parsed from a NUL-terminated copy: a number at its end
    // cannot read on into tensor data or past the mapping
    const std::string hdr(reinterpret_cast<const char *>(b + 8), static_cast<size_t>(hlen));
    JParser jp{hdr.c_str(), hdr.c_str() + hdr.size()};
    JVal root = jp.value();
    XE_REQUIRE(root.t == JVal::OBJ, "safetensors header: object expected");
    const uint8_t *data0 = b + 8 + hlen;
    const size_t data_size = size - 8 - hlen;
    for (const auto &kv : root.obj) {
      if (kv.first == "__metadata__") {
        for (const auto &m : kv.second.obj)
          if (m.second.t == JVal::STR) meta[m.first] = m.second.str;
        continue;
      }
      const JVal &t = kv.second;
      const JVal *dt = t.get("dtype"), *sh = t.get("shape"), *off = t.get("data_offsets");
      XE_REQUIRE(dt && dt->t == JVal::STR && sh && sh->t == JVal::ARR && off && off->t == JVal::ARR &&
                     off->arr.size() == 2,
                 "safetensors header: tensor " + kv.first + " lacks dtype / shape / data_offsets");
      TensorRef r;
      r.dtype = dt->str;
      size_t n = 1;
      for (const auto &d : sh->arr) {
        const size_t dim = json_index(d, "shape of " + kv.first);
        XE_REQUIRE(dim == 0 || n <= SIZE_MAX / dim, "safetensors header: shape of " + kv.first + " overflows");
        r.shape.push_back(static_cast<int64_t>(dim));
        n *= dim;
      }
      const size_t o0 = json_index(off->arr[0], "data_offsets of " + kv.first);
      const size_t o1 = json_index(off->arr[1], "data_offsets of " + kv.first);
      XE_REQUIRE(o0 <= o1 && o1 <= data_size, "safetensors header: data_offsets of " + kv.first + " out of range");
      const size_t esz = r.dtype == "F32" ? 4 : (r.dtype == "BF16" || r.dtype == "F16") ? 2 : 0;
      if (esz)
        XE_REQUIRE(n <= SIZE_MAX / esz && o1 - o0 == n * esz,
                   "safetensors: byte size of " + kv.first + " does not match its shape");
      r.data = data0 + o0;
      r.bytes = o1 - o0;
      tensors[kv.first] = r;
    }
  }
  ~StFile() {
    if (map && map != MAP_FAILED) ::munmap(map, size);
    if (fd >= 0) ::close(fd);
  }
  StFile(const StFile &) = delete;
  StFile &operator=(const StFile &) = delete;
};

float half_to_f32(uint16_t h) {
  const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
  const int e = (h >> 10) & 0x1f;
  uint32_t m = h & 0x3ffu;
  uint32_t bits;
  if (e == 0x1f) {
    bits = sign | 0x7f800000u | (m << 13);
  } else if (e == 0) {
    if (m == 0) {
      bits = sign;
    } else {  // subnormal: normalise
      int ee = -1;
      do {
        m <<= 1;
        ee++;
      } while (!(m & 0x400u));
      bits = sign | static_cast<uint32_t>(127 - 15 - ee) << 23 | (m & 0x3ffu) << 13;
    }
  } else {
    bits = sign | static_cast<uint32_t>(e - 15 + 127) << 23 | m << 13;
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

std::vector<float> to_f32(const TensorRef &r, const std::string &name) {
  size_t n = 1;
  for (auto d : r.shape) n *= static_cast<size_t>(d);
  std::vector<float> out(n);
  if (r.dtype == "F32") {
    std::memcpy(out.data(), r.data, n * 4);
  } else if (r.dtype == "BF16") {
    for (size_t i = 0; i < n; i++) {
      const uint32_t b = static_cast<uint32_t>(r.data[2 * i] | r.data[2 * i + 1] << 8) << 16;
      std::memcpy(&out[i], &b, 4);
    }
  } else if (r.dtype == "F16") {
    for (size_t i = 0; i < n; i++) out[i] = half_to_f32(static_cast<uint16_t>(r.data[2 * i] | r.data[2 * i + 1] << 8));
  } else {
    fail("safetensors: tensor " + name + " has dtype " + r.dtype + " (F32 / BF16 / F16 supported)");
  }
  return out;
}

// ---------------------------------------------------------------------------
// names -> (tensor kind, layer)
// ---------------------------------------------------------------------------
struct Target {
  int kind = -1;
  int layer = -1;
  bool transposed = false;  // stored [in, out]
};

// "prefix{i}.rest" / "prefix{i}/rest" -> (i, rest)
bool split_layer(const std::string &n, const std::string &prefix, char sep, int &layer, std::string &rest) {
  if (n.compare(0, prefix.size(), prefix) != 0) return false;
  size_t i = prefix.size(), j = i;
  while (j < n.size() && std::isdigit(static_cast<unsigned char>(n[j]))) j++;
  if (j == i || j >= n.size() || n[j] != sep) return false;
  layer = std::atoi(n.substr(i, j - i).c_str());
  rest = n.substr(j + 1);
  return true;
}

// The reference's baked OPT arena (arch/opt.rs:1-20): linears transposed
// [in, out], vectors verbatim, lm_head transposed (tied: not loaded).
bool map_arena_opt(const std::string &n, Target &t) {
  static const std::map<std::string, int> glob = {{"embed_tokens", XE_T_TOK_EMB},
                                                  {"embed_positions", XE_T_POS_EMB},
                                                  {"ln_final.weight", XE_T_LNF_W},
                                                  {"ln_final.bias", XE_T_LNF_B}};
  static const std::map<std::string, std::pair<int, bool>> per = {
      {"q.weight", {XE_T_Q_W, true}},     {"q.bias", {XE_T_Q_B, false}},
      {"k.weight", {XE_T_K_W, true}},     {"k.bias", {XE_T_K_B, false}},
      {"v.weight", {XE_T_V_W, true}},     {"v.bias", {XE_T_V_B, false}},
      {"out.weight", {XE_T_O_W, true}},   {"out.bias", {XE_T_O_B, false}},
      {"ln_self.weight", {XE_T_LN1_W, false}}, {"ln_self.bias", {XE_T_LN1_B, false}},
      {"fc1.weight", {XE_T_FC1_W, true}}, {"fc1.bias", {XE_T_FC1_B, false}},
      {"fc2.weight", {XE_T_FC2_W, true}}, {"fc2.bias", {XE_T_FC2_B, false}},
      {"ln_ffn.weight", {XE_T_LN2_W, false}}, {"ln_ffn.bias", {XE_T_LN2_B, false}}};
  auto g = glob.find(n);
  if (g != glob.end()) {
    t.kind = g->second;
    t.layer = -1;
    return true;
  }
  int l;
  std::string rest;
  if (!split_layer(n, "L", '/', l, rest)) return false;
  auto p = per.find(rest);
  if (p == per.end()) return false;
  t.kind = p->second.first;
  t.transposed = p->second.second;
  t.layer = l;
  return true;
}

// Hugging Face checkpoint names ([out, in] linears) of the three decoders:
// OPTForCausalLM (model.decoder.*), Whisper's decoder (model.decoder.*, with
// encoder_attn), Gemma3ForCausalLM (model.layers.*; a multimodal checkpoint's
// model.language_model.* is accepted too).
bool map_hf(int family, std::string n, Target &t) {
  if (n.compare(0, 21, "model.language_model.") == 0) n = "model." + n.substr(21);
  if (family == XE_GEMMA3) {
    static const std::map<std::string, int> glob = {{"model.embed_tokens.weight", XE_T_TOK_EMB},
                                                    {"model.norm.weight", XE_T_LNF_W}};
    static const std::map<std::string, int> per = {
        {"self_attn.q_proj.weight", XE_T_Q_W},        {"self_attn.k_proj.weight", XE_T_K_W},
        {"self_attn.v_proj.weight", XE_T_V_W},        {"self_attn.o_proj.weight", XE_T_O_W},
        {"self_attn.q_norm.weight", XE_T_QNORM_W},    {"self_attn.k_norm.weight", XE_T_KNORM_W},
        {"input_layernorm.weight", XE_T_LN1_W},       {"post_attention_layernorm.weight", XE_T_POST_ATTN_W},
        {"pre_feedforward_layernorm.weight", XE_T_LN2_W}, {"post_feedforward_layernorm.weight", XE_T_POST_FFN_W},
        {"mlp.gate_proj.weight", XE_T_FC1_W},         {"mlp.up_proj.weight", XE_T_UP_W},
        {"mlp.down_proj.weight", XE_T_FC2_W}};
    auto g = glob.find(n);
    if (g != glob.end()) {
      t.kind = g->second;
      return true;
    }
    int l;
    std::string rest;
    if (!split_layer(n, "model.layers.", '.', l, rest)) return false;
    auto p = per.find(rest);
    if (p == per.end()) return false;
    t.kind = p->second;
    t.layer = l;
    return true;
  }
  const bool wh = family == XE_WHISPER;
  static const std::map<std::string, int> glob_opt = {
      {"model.decoder.embed_tokens.weight", XE_T_TOK_EMB},
      {"model.decoder.embed_positions.weight", XE_T_POS_EMB},
      {"model.decoder.final_layer_norm.weight", XE_T_LNF_W},
      {"model.decoder.final_layer_norm.bias", XE_T_LNF_B}};
  static const std::map<std::string, int> glob_wh = {
      {"model.decoder.embed_tokens.weight", XE_T_TOK_EMB},
      {"model.decoder.embed_positions.weight", XE_T_POS_EMB},
      {"model.decoder.layer_norm.weight", XE_T_LNF_W},
      {"model.decoder.layer_norm.bias", XE_T_LNF_B}};
  static const std::map<std::string, int> per = {
      {"self_attn.q_proj.weight", XE_T_Q_W},     {"self_attn.q_proj.bias", XE_T_Q_B},
      {"self_attn.k_proj.weight", XE_T_K_W},     {"self_attn.k_proj.bias", XE_T_K_B},
      {"self_attn.v_proj.weight", XE_T_V_W},     {"self_attn.v_proj.bias", XE_T_V_B},
      {"self_attn.out_proj.weight", XE_T_O_W},   {"self_attn.out_proj.bias", XE_T_O_B},
      {"self_attn_layer_norm.weight", XE_T_LN1_W}, {"self_attn_layer_norm.bias", XE_T_LN1_B},
      {"encoder_attn.q_proj.weight", XE_T_XQ_W}, {"encoder_attn.q_proj.bias", XE_T_XQ_B},
      {"encoder_attn.k_proj.weight", XE_T_XK_W},
      {"encoder_attn.v_proj.weight", XE_T_XV_W}, {"encoder_attn.v_proj.bias", XE_T_XV_B},
      {"encoder_attn.out_proj.weight", XE_T_XO_W}, {"encoder_attn.out_proj.bias", XE_T_XO_B},
      {"encoder_attn_layer_norm.weight", XE_T_LNX_W}, {"encoder_attn_layer_norm.bias", XE_T_LNX_B},
      {"fc1.weight", XE_T_FC1_W},                {"fc1.bias", XE_T_FC1_B},
      {"fc2.weight", XE_T_FC2_W},                {"fc2.bias", XE_T_FC2_B},
      {"final_layer_norm.weight", XE_T_LN2_W},   {"final_layer_norm.bias", XE_T_LN2_B}};
  const auto &glob = wh ? glob_wh : glob_opt;
  auto g = glob.find(n);
  if (g != glob.end()) {
    t.kind = g->second;
    return true;
  }
  int l;
  std::string rest;
  if (!split_layer(n, "model.decoder.layers.", '.', l, rest)) return false;
  auto p = per.find(rest);
  if (p == per.end()) return false;
  t.kind = p->second;
  t.layer = l;
  return true;
}

// Tied output matrices a checkpoint may carry instead of (or beside) the
// token embedding ([vocab, d], untransposed): OPT's lm_head (arch/opt.rs:18-20
// rebuilds embed_tokens from it), Whisper's proj_out, Gemma's lm_head.
bool is_tied_head(const std::string &n) { return n == "lm_head.weight" || n == "proj_out.weight"; }

struct Plan {
  std::vector<std::pair<std::string, Target>> items;
  std::vector<std::string> skipped;
  bool arena = false;
};

// Which tensors of the file feed which (kind, layer).  shape_of(kind, layer,
// rows, cols) gives the decoder's expected [out, in] shape (false: the family
// has no such tensor).
template <typename ShapeOf>
Plan plan_file(const StFile &f, int family, int n_layers, ShapeOf shape_of) {
  Plan pl;
  auto a = f.meta.find("arch");
  pl.arena = a != f.meta.end() && f.meta.count("format_version");
  if (pl.arena) {
    XE_REQUIRE(family == XE_OPT && a->second == "opt",
               "arena arch \"" + a->second + "\" has no decoder mapping for this model family (baked OPT arenas "
               "only; load Hugging Face checkpoints for Whisper / Gemma-3)");
    XE_REQUIRE(f.meta.at("format_version") == "1",
               "arena format_version " + f.meta.at("format_version") + " != 1 (rebake)");
  }
  std::set<std::pair<int, int>> have;
  std::string tied;
  for (const auto &kv : f.tensors) {
    Target t;
    const bool ok = pl.arena ? map_arena_opt(kv.first, t) : map_hf(family, kv.first, t);
    int rows = 0, cols = 0;
    if (!ok || t.layer >= n_layers || !shape_of(t.kind, t.layer, rows, cols)) {
      if (is_tied_head(kv.first) && !pl.arena) tied = kv.first;
      pl.skipped.push_back(kv.first);
      continue;
    }
    XE_REQUIRE(have.insert({t.kind, t.layer}).second, "two tensors of the file map to " + kv.first);
    pl.items.push_back({kv.first, t});
  }
  // OPT / Whisper checkpoints may omit the tied embedding (arch/opt.rs:18-20)
  if (!have.count({XE_T_TOK_EMB, -1}) && !tied.empty()) {
    Target t;
    t.kind = XE_T_TOK_EMB;
    pl.items.push_back({tied, t});
    have.insert({XE_T_TOK_EMB, -1});
    for (size_t i = 0; i < pl.skipped.size(); i++)
      if (pl.skipped[i] == tied) {
        pl.skipped.erase(pl.skipped.begin() + static_cast<long>(i));
        break;
      }
  }
  // every tensor the model needs (the synthetic encoder output aside)
  std::string missing;
  for (int layer = -1; layer < n_layers; layer++)
    for (int kind = 0; kind < XE_T_COUNT; kind++) {
      int rows = 0, cols = 0;
      if (kind == XE_T_ENC_OUT || !shape_of(kind, layer, rows, cols)) continue;
      if (!have.count({kind, layer}))
        missing += (missing.empty() ? "" : ", ") + std::string("kind ") + std::to_string(kind) + " layer " +
                   std::to_string(layer);
    }
  XE_REQUIRE(missing.empty(), "weight file lacks tensors the model needs: " + missing);
  return pl;
}

}  // namespace

}  // namespace xe

using xe::StFile;

extern "C" {

int xe_decoder_load_safetensors(xe_decoder *d, const char *path) {
  try {
    XE_REQUIRE(d, "null decoder");
    StFile f(path);
    xe_model_config c{};
    XE_REQUIRE(xe_decoder_config(d, &c) == 0, xe_last_error());
    auto shape_of = [&](int kind, int layer, int &rows, int &cols) {
      return xe_model_tensor_shape(&c, kind, layer, &rows, &cols) == 0;
    };
    xe::Plan pl = xe::plan_file(f, c.family, c.n_layers, shape_of);
    for (const auto &it : pl.items) {
      const xe::TensorRef &r = f.tensors.at(it.first);
      const xe::Target &t = it.second;
      int rows = 0, cols = 0;
      shape_of(t.kind, t.layer, rows, cols);
      size_t n = 1;
      for (auto v : r.shape) n *= static_cast<size_t>(v);
      XE_REQUIRE(n == static_cast<size_t>(rows) * cols,
                 it.first + ": " + std::to_string(n) + " elements, the model needs " + std::to_string(rows) + " x " +
                     std::to_string(cols));
      std::vector<float> v = xe::to_f32(r, it.first);
      if (t.transposed) {  // [in, out] -> [out, in]
        XE_REQUIRE(r.shape.size() == 2 && r.shape[0] == cols && r.shape[1] == rows,
                   it.first + ": expected an [in, out] = [" + std::to_string(cols) + ", " + std::to_string(rows) +
                       "] matrix");
        std::vector<float> tr(v.size());
        for (int i = 0; i < cols; i++)
          for (int o = 0; o < rows; o++) tr[static_cast<size_t>(o) * cols + i] = v[static_cast<size_t>(i) * rows + o];
        v.swap(tr);
      }
      XE_REQUIRE(xe_decoder_set_tensor(d, t.kind, t.layer, v.data(), v.size()) == 0,
                 it.first + ": " + xe_last_error());
    }
    return static_cast<int>(pl.items.size());
  } catch (const std::exception &e) {
    xe::set_error(e.what());
    return -1;
  } catch (...) {
    xe::set_error("unknown error");
    return -1;
  }
}

int xe_safetensors_plan(const char *path, const xe_model_config *cfg, char *report, int cap) {
  try {
    XE_REQUIRE(cfg, "null config");
    StFile f(path);
    auto shape_of = [&](int kind, int layer, int &rows, int &cols) {
      return xe_model_tensor_shape(cfg, kind, layer, &rows, &cols) == 0;
    };
    xe::Plan pl = xe::plan_file(f, cfg->family, cfg->n_layers, shape_of);
    if (report && cap > 0) {
      std::string s = pl.arena ? "arena" : "hf";
      for (const auto &it : pl.items)
        s += "\n" + it.first + " -> " + std::to_string(it.second.kind) + " " + std::to_string(it.second.layer) +
             (it.second.transposed ? " T" : "");
      for (const auto &n : pl.skipped) s += "\n" + n + " -> skipped";
      std::snprintf(report, static_cast<size_t>(cap), "%s", s.c_str());
    }
    return static_cast<int>(pl.items.size());
  } catch (const std::exception &e) {
    xe::set_error(e.what());
    return -1;
  } catch (...) {
    xe::set_error("unknown error");
    return -1;
  }
}

}  // extern "C"
