// Safetensors reader for GPT-OSS MXFP4 checkpoints — the reference's ShardReader
// (weights.rs:103-139: a u64 little-endian header length, that many bytes of JSON mapping each
// tensor name to {dtype, shape, data_offsets}, then the data; offsets count from the data's
// start) and the per-layer tensor names of load_weights (weights.rs:228-346). Host code only:
// the shards are memory-mapped and the expert tensors are handed to moe_preload_layer straight
// from the mapping (no copy of the 13 MB-per-expert blocks); biases and the router bias are
// widened from bf16 to f32 (exact), the router weight stays bf16 bits, as moe_preload_router
// takes it.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cctype>
#include <cerrno>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "../../include/mxfp4_moe.h"

namespace moe {
int api_fail(int code, const char *msg);
int ctx_dims(const moe_ctx *c, size_t *H, size_t *I);
}

namespace {

int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  return moe::api_fail(code, buf);
}

struct TensorInfo {
  std::string dtype;
  std::vector<uint64_t> shape;
  uint64_t begin = 0, end = 0;  // byte range in the file
};

// A read-only mapping of one shard and its parsed header.
struct Shard {
  std::string path;
  const uint8_t *base = nullptr;
  size_t size = 0;
  std::map<std::string, TensorInfo> tensors;
  Shard() = default;
  Shard(const Shard &) = delete;
  Shard &operator=(const Shard &) = delete;
  ~Shard() {
    if (base) munmap(const_cast<uint8_t *>(base), size);
  }
};

// Minimal JSON reader for the header: objects, arrays, strings (with escapes), numbers,
// true/false/null. Numbers used as shapes or offsets must be non-negative integers.
struct Json {
  const char *p, *e;
  std::string err;
  bool fail_at(const char *what) {
    if (err.empty()) err = std::string(what) + " (" + std::to_string((long)(e - p)) + " header bytes left)";
    return false;
  }
  void ws() {
    while (p < e && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
  }
  bool lit(char c) {
    ws();
    if (p < e && *p == c) {
      p++;
      return true;
    }
    return false;
  }
  bool str(std::string &out) {
    ws();
    if (p >= e || *p != '"') return fail_at("expected a string");
    p++;
    out.clear();
    while (p < e && *p != '"') {
      if (*p == '\\') {
        if (++p >= e) return fail_at("unterminated escape");
        const char c = *p++;
        switch (c) {
          case '"': out += '"'; break;
          case '\\': out += '\\'; break;
          case '/': out += '/'; break;
          case 'b': out += '\b'; break;
          case 'f': out += '\f'; break;
          case 'n': out += '\n'; break;
          case 'r': out += '\r'; break;
          case 't': out += '\t'; break;
          case 'u': {  // kept as UTF-8 for the basic plane; names here are ASCII
            if (e - p < 4) return fail_at("short \\u escape");
            unsigned v = 0;
            for (int i = 0; i < 4; i++) {
              const char h = *p++;
              v = v * 16 + (h >= '0' && h <= '9' ? h - '0' : h >= 'a' && h <= 'f' ? h - 'a' + 10 : h >= 'A' && h <= 'F' ? h - 'A' + 10 : 99);
              if (v > 0xFFFF) return fail_at("bad \\u escape");
            }
            if (v < 0x80) {
              out += (char)v;
            } else if (v < 0x800) {
              out += (char)(0xC0 | (v >> 6));
              out += (char)(0x80 | (v & 0x3F));
            } else {
              out += (char)(0xE0 | (v >> 12));
              out += (char)(0x80 | ((v >> 6) & 0x3F));
              out += (char)(0x80 | (v & 0x3F));
            }
            break;
          }
          default: return fail_at("bad escape");
        }
      } else {
        out += *p++;
      }
    }
    if (p >= e) return fail_at("unterminated string");
    p++;
    return true;
  }
  bool uint(uint64_t &v) {
    ws();
    if (p >= e || *p < '0' || *p > '9') return fail_at("expected a non-negative integer");
    v = 0;
    while (p < e && *p >= '0' && *p <= '9') {
      const uint64_t d = (uint64_t)(*p++ - '0');
      if (v > (UINT64_MAX - d) / 10) return fail_at("integer overflow");
      v = v * 10 + d;
    }
    if (p < e && (*p == '.' || *p == 'e' || *p == 'E')) return fail_at("expected an integer");
    return true;
  }
  bool skip() {  // any value
    ws();
    if (p >= e) return fail_at("unexpected end");
    if (*p == '"') {
      std::string s;
      return str(s);
    }
    if (*p == '{' || *p == '[') {
      const char close = *p == '{' ? '}' : ']';
      const bool obj = *p == '{';
      p++;
      if (lit(close)) return true;
      do {
        if (obj) {
          std::string k;
          if (!str(k) || !lit(':')) return fail_at("bad object");
        }
        if (!skip()) return false;
      } while (lit(','));
      return lit(close) || fail_at("unterminated container");
    }
    const char *s = p;
    while (p < e && (isalnum((unsigned char)*p) || *p == '-' || *p == '+' || *p == '.')) p++;
    return p > s || fail_at("unexpected character");
  }
  bool uint_array(std::vector<uint64_t> &v) {
    v.clear();
    if (!lit('[')) return fail_at("expected an array");
    if (lit(']')) return true;
    do {
      uint64_t x;
      if (!uint(x)) return false;
      v.push_back(x);
    } while (lit(','));
    return lit(']') || fail_at("unterminated array");
  }
  // data0: file offset of the data section; data_len: its length (file size - data0). Offsets are
  // checked against data_len before data0 is added, so no sum can wrap.
  bool tensor(TensorInfo &t, uint64_t data0, uint64_t data_len) {
    if (!lit('{')) return fail_at("expected a tensor entry");
    bool have_d = false, have_s = false, have_o = false;
    if (!lit('}')) {
      do {
        std::string k;
        if (!str(k) || !lit(':')) return fail_at("bad tensor entry");
        if (k == "dtype") {
          if (!str(t.dtype)) return false;
          have_d = true;
        } else if (k == "shape") {
          if (!uint_array(t.shape)) return false;
          have_s = true;
        } else if (k == "data_offsets") {
          std::vector<uint64_t> o;
          if (!uint_array(o)) return false;
          if (o.size() != 2 || o[1] < o[0]) return fail_at("data_offsets must be [begin, end]");
          if (o[1] > data_len) return fail_at("data_offsets run past the end of the file");
          t.begin = data0 + o[0];
          t.end = data0 + o[1];
          have_o = true;
        } else if (!skip()) {
          return false;
        }
      } while (lit(','));
      if (!lit('}')) return fail_at("unterminated tensor entry");
    }
    return (have_d && have_s && have_o) || fail_at("tensor entry without dtype, shape or data_offsets");
  }
};

int open_shard(const char *path, Shard &sh) {
  sh.path = path ? path : "";
  const int fd = path ? ::open(path, O_RDONLY) : -1;
  if (fd < 0) return fail(MOE_ERR_IO, "cannot open %s: %s", sh.path.c_str(), strerror(errno));
  struct stat st;
  if (fstat(fd, &st) != 0 || st.st_size < 8) {
    ::close(fd);
    return fail(MOE_ERR_IO, "%s: not a safetensors file (shorter than its 8-byte header length)", path);
  }
  void *m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (m == MAP_FAILED) return fail(MOE_ERR_IO, "cannot map %s: %s", path, strerror(errno));
  sh.base = (const uint8_t *)m;
  sh.size = (size_t)st.st_size;
  uint64_t n = 0;
  for (int i = 7; i >= 0; i--) n = (n << 8) | sh.base[i];
  if (n > sh.size - 8) return fail(MOE_ERR_IO, "%s: header length %llu runs past the file", path, (unsigned long long)n);
  Json j{(const char *)sh.base + 8, (const char *)sh.base + 8 + n, {}};
  const uint64_t data0 = 8 + n;
  bool ok = j.lit('{');
  if (ok && !j.lit('}')) {
    do {
      std::string name;
      if (!(ok = j.str(name) && j.lit(':'))) break;
      if (name == "__metadata__") {
        if (!(ok = j.skip())) break;
        continue;
      }
      TensorInfo t;
      if (!(ok = j.tensor(t, data0, sh.size - data0))) {
        j.err = "tensor " + name + ": " + j.err;
        break;
      }
      sh.tensors[name] = t;
    } while (j.lit(','));
    if (ok) ok = j.lit('}');
  }
  if (!ok) return fail(MOE_ERR_IO, "%s: bad header: %s", path, j.err.empty() ? "expected an object" : j.err.c_str());
  return MOE_OK;
}

size_t dtype_bytes(const std::string &d) {
  if (d == "U8" || d == "I8" || d == "BOOL" || d == "F8_E4M3" || d == "F8_E5M2") return 1;
  if (d == "BF16" || d == "F16" || d == "I16" || d == "U16") return 2;
  if (d == "F32" || d == "I32" || d == "U32") return 4;
  if (d == "F64" || d == "I64" || d == "U64") return 8;
  return 0;
}

// The first shard holding `name` (the reference's get_tensor_bytes, weights.rs:216-224), checked
// against the expected dtype and shape.
int find(const std::vector<Shard> &shards, const std::string &name, const char *dtype,
         const std::vector<uint64_t> &shape, const uint8_t **data) {
  for (const Shard &sh : shards) {
    auto it = sh.tensors.find(name);
    if (it == sh.tensors.end()) continue;
    const TensorInfo &t = it->second;
    if (t.dtype != dtype) return fail(MOE_ERR_INVALID, "%s: dtype %s, expected %s", name.c_str(), t.dtype.c_str(), dtype);
    if (t.shape != shape) {
      std::string got, want;
      for (uint64_t v : t.shape) got += std::to_string(v) + ",";
      for (uint64_t v : shape) want += std::to_string(v) + ",";
      return fail(MOE_ERR_INVALID, "%s: shape [%s], expected [%s]", name.c_str(), got.c_str(), want.c_str());
    }
    uint64_t n = dtype_bytes(t.dtype);
    for (uint64_t v : t.shape) n *= v;
    if (t.end - t.begin != n)
      return fail(MOE_ERR_INVALID, "%s: %llu data bytes for %llu expected", name.c_str(),
                  (unsigned long long)(t.end - t.begin), (unsigned long long)n);
    *data = sh.base + t.begin;
    return MOE_OK;
  }
  return fail(MOE_ERR_INVALID, "tensor %s not found in any shard", name.c_str());
}

std::vector<float> bf16_to_f32(const uint8_t *p, size_t n) {  // exact: the bf16 bits are the top half
  std::vector<float> out(n);
  for (size_t i = 0; i < n; i++) {
    const uint32_t u = (uint32_t)(p[2 * i] | (p[2 * i + 1] << 8)) << 16;
    std::memcpy(&out[i], &u, 4);
  }
  return out;
}

}  // namespace

extern "C" int moe_safetensors_find(const char *path, const char *name, char *dtype, size_t dtype_cap,
                                    uint64_t *shape, size_t shape_cap, size_t *rank, uint64_t *begin,
                                    uint64_t *end) {
  if (!path || !name || !rank || !begin || !end) return fail(MOE_ERR_INVALID, "null argument");
  Shard sh;
  if (int r = open_shard(path, sh)) return r;
  auto it = sh.tensors.find(name);
  if (it == sh.tensors.end()) return fail(MOE_ERR_INVALID, "tensor %s not in %s", name, path);
  const TensorInfo &t = it->second;
  if (dtype && dtype_cap) {
    std::snprintf(dtype, dtype_cap, "%s", t.dtype.c_str());
  }
  *rank = t.shape.size();
  for (size_t i = 0; i < t.shape.size() && i < shape_cap && shape; i++) shape[i] = t.shape[i];
  *begin = t.begin;
  *end = t.end;
  return MOE_OK;
}

extern "C" int moe_load_safetensors_layer(moe_ctx *ctx, const char *const *shard_paths, size_t n_shards,
                                          size_t layer, size_t n_experts, float rms_norm_eps) {
  size_t hidden = 0, inter = 0;
  if (int r = moe::ctx_dims(ctx, &hidden, &inter)) return r;
  if (!shard_paths || !n_shards) return fail(MOE_ERR_INVALID, "no shards");
  if (!n_experts) return fail(MOE_ERR_INVALID, "no experts");
  std::vector<Shard> shards(n_shards);
  for (size_t i = 0; i < n_shards; i++)
    if (int r = open_shard(shard_paths[i], shards[i])) return r;
  const std::string lp = "model.layers." + std::to_string(layer) + ".mlp.";
  const uint64_t E = n_experts, H = hidden, I = inter;
  const uint8_t *gub, *gus, *gubias, *db, *ds, *dbias, *rw, *rb;
  if (int r = find(shards, lp + "experts.gate_up_proj_blocks", "U8", {E, 2 * I, H / 32, 16}, &gub)) return r;
  if (int r = find(shards, lp + "experts.gate_up_proj_scales", "U8", {E, 2 * I, H / 32}, &gus)) return r;
  if (int r = find(shards, lp + "experts.gate_up_proj_bias", "BF16", {E, 2 * I}, &gubias)) return r;
  if (int r = find(shards, lp + "experts.down_proj_blocks", "U8", {E, H, I / 32, 16}, &db)) return r;
  if (int r = find(shards, lp + "experts.down_proj_scales", "U8", {E, H, I / 32}, &ds)) return r;
  if (int r = find(shards, lp + "experts.down_proj_bias", "BF16", {E, H}, &dbias)) return r;
  if (int r = find(shards, lp + "router.weight", "BF16", {E, H}, &rw)) return r;
  if (int r = find(shards, lp + "router.bias", "BF16", {E}, &rb)) return r;
  const std::vector<float> gb = bf16_to_f32(gubias, E * 2 * I), dbf = bf16_to_f32(dbias, E * H),
                           rbf = bf16_to_f32(rb, E);
  if (int r = moe_preload_layer(ctx, layer, n_experts, gub, gus, gb.data(), db, ds, dbf.data())) return r;
  std::vector<uint16_t> rwb(E * H);
  std::memcpy(rwb.data(), rw, rwb.size() * 2);  // bf16 bits, little-endian as stored
  if (int r = moe_preload_router(ctx, layer, n_experts, rwb.data(), rbf.data())) return r;
  // the post-attention RMSNorm weight, when the shards hold it (weights.rs:267-268)
  const std::string nn = "model.layers." + std::to_string(layer) + ".post_attention_layernorm.weight";
  for (const Shard &sh : shards)
    if (sh.tensors.count(nn)) {
      const uint8_t *g;
      if (int r = find(shards, nn, "BF16", {H}, &g)) return r;
      const std::vector<float> gf = bf16_to_f32(g, H);
      return moe_preload_norm(ctx, layer, gf.data(), rms_norm_eps);
    }
  return MOE_OK;
}
