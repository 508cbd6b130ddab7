// checkpoint.cpp -- FORGEMODEL1 checkpoint reader (host side) for the HIP session.
//
// Format (src/LLM.Core/Checkpoint/Checkpoint.cs:143-166 writer, 174-250 reader):
//   "FORGEMODEL1" | int32 LE json length | UTF-8 JSON header | every registry
//   tensor as little-endian fp32 in registry order | (Training.HasOptimizerState:
//   Adam M then V per tensor) | SHA-256 of everything before it (32 bytes).
// The header is System.Text.Json's default serialization of the reference's
// Header class (PascalCase property names, case-sensitive, unknown properties
// ignored).  Validation order and messages follow Checkpoint.LoadCore.
//
// SHA-256 follows FIPS 180-4 (section 6.2); the JSON reader is a small
// recursive-descent parser of RFC 8259 values.
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <vector>

namespace fh {

// ---------------------------------------------------------------- SHA-256 --
struct Sha256 {
  uint32_t h[8];
  uint64_t len = 0;  // bytes hashed
  uint8_t buf[64];
  int nbuf = 0;

  Sha256() {
    static const uint32_t init[8] = {0x6a09e667u, 0xbb67ae85u, 0x3c6ef372u, 0xa54ff53au,
                                     0x510e527fu, 0x9b05688cu, 0x1f83d9abu, 0x5be0cd19u};
    memcpy(h, init, sizeof h);
  }
  static uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }
  void block(const uint8_t* p) {
    // round constants: first 32 bits of the fractional parts of the cube roots of the first 64 primes
    static const uint32_t k[64] = {
        0x428a2f98u, 0x71374491u, 0xb5c0fbcfu, 0xe9b5dba5u, 0x3956c25bu, 0x59f111f1u, 0x923f82a4u, 0xab1c5ed5u,
        0xd807aa98u, 0x12835b01u, 0x243185beu, 0x550c7dc3u, 0x72be5d74u, 0x80deb1feu, 0x9bdc06a7u, 0xc19bf174u,
        0xe49b69c1u, 0xefbe4786u, 0x0fc19dc6u, 0x240ca1ccu, 0x2de92c6fu, 0x4a7484aau, 0x5cb0a9dcu, 0x76f988dau,
        0x983e5152u, 0xa831c66du, 0xb00327c8u, 0xbf597fc7u, 0xc6e00bf3u, 0xd5a79147u, 0x06ca6351u, 0x14292967u,
        0x27b70a85u, 0x2e1b2138u, 0x4d2c6dfcu, 0x53380d13u, 0x650a7354u, 0x766a0abbu, 0x81c2c92eu, 0x92722c85u,
        0xa2bfe8a1u, 0xa81a664bu, 0xc24b8b70u, 0xc76c51a3u, 0xd192e819u, 0xd6990624u, 0xf40e3585u, 0x106aa070u,
        0x19a4c116u, 0x1e376c08u, 0x2748774cu, 0x34b0bcb5u, 0x391c0cb3u, 0x4ed8aa4au, 0x5b9cca4fu, 0x682e6ff3u,
        0x748f82eeu, 0x78a5636fu, 0x84c87814u, 0x8cc70208u, 0x90befffau, 0xa4506cebu, 0xbef9a3f7u, 0xc67178f2u};
    uint32_t w[64];
    for (int t = 0; t < 16; t++)
      w[t] = (uint32_t)p[4 * t] << 24 | (uint32_t)p[4 * t + 1] << 16 | (uint32_t)p[4 * t + 2] << 8 | p[4 * t + 3];
    for (int t = 16; t < 64; t++) {
      const uint32_t s0 = rotr(w[t - 15], 7) ^ rotr(w[t - 15], 18) ^ (w[t - 15] >> 3);
      const uint32_t s1 = rotr(w[t - 2], 17) ^ rotr(w[t - 2], 19) ^ (w[t - 2] >> 10);
      w[t] = w[t - 16] + s0 + w[t - 7] + s1;
    }
    uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
    for (int t = 0; t < 64; t++) {
      const uint32_t S1 = rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25);
      const uint32_t ch = (e & f) ^ (~e & g);
      const uint32_t t1 = hh + S1 + ch + k[t] + w[t];
      const uint32_t S0 = rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22);
      const uint32_t maj = (a & b) ^ (a & c) ^ (b & c);
      const uint32_t t2 = S0 + maj;
      hh = g;
      g = f;
      f = e;
      e = d + t1;
      d = c;
      c = b;
      b = a;
      a = t1 + t2;
    }
    h[0] += a;
    h[1] += b;
    h[2] += c;
    h[3] += d;
    h[4] += e;
    h[5] += f;
    h[6] += g;
    h[7] += hh;
  }
  void update(const void* data, size_t n) {
    const uint8_t* p = static_cast<const uint8_t*>(data);
    len += n;
    if (nbuf) {
      const size_t take = n < (size_t)(64 - nbuf) ? n : (size_t)(64 - nbuf);
      memcpy(buf + nbuf, p, take);
      nbuf += (int)take;
      p += take;
      n -= take;
      if (nbuf == 64) {
        block(buf);
        nbuf = 0;
      }
    }
    for (; n >= 64; n -= 64, p += 64) block(p);
    if (n) {
      memcpy(buf, p, n);
      nbuf = (int)n;
    }
  }
  void final(uint8_t out[32]) {
    const uint64_t bits = len * 8;
    const uint8_t pad = 0x80;
    update(&pad, 1);
    const uint8_t zero[64] = {0};
    update(zero, (size_t)((nbuf <= 56) ? 56 - nbuf : 120 - nbuf));
    uint8_t lb[8];
    for (int i = 0; i < 8; i++) lb[i] = (uint8_t)(bits >> (56 - 8 * i));
    update(lb, 8);
    for (int i = 0; i < 8; i++)
      for (int j = 0; j < 4; j++) out[4 * i + j] = (uint8_t)(h[i] >> (24 - 8 * j));
  }
};

void sha256(const void* data, size_t n, uint8_t out[32]) {
  Sha256 s;
  s.update(data, n);
  s.final(out);
}

// ------------------------------------------------------------------- JSON --
struct Json {
  enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
  bool b = false;
  double num = 0;
  std::string str;
  std::vector<Json> arr;
  std::vector<std::pair<std::string, Json>> obj;
  const Json* get(const char* key) const {
    for (auto& kv : obj)
      if (kv.first == key) return &kv.second;
    return nullptr;
  }
};

struct JsonParser {
  const char* p;
  const char* end;
  int depth = 0;
  void ws() {
    while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
  }
  bool lit(const char* s) {
    const size_t n = strlen(s);
    if ((size_t)(end - p) < n || memcmp(p, s, n) != 0) return false;
    p += n;
    return true;
  }
  static void utf8(std::string& o, uint32_t cp) {
    if (cp < 0x80) {
      o += (char)cp;
    } else if (cp < 0x800) {
      o += (char)(0xC0 | (cp >> 6));
      o += (char)(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      o += (char)(0xE0 | (cp >> 12));
      o += (char)(0x80 | ((cp >> 6) & 0x3F));
      o += (char)(0x80 | (cp & 0x3F));
    } else {
      o += (char)(0xF0 | (cp >> 18));
      o += (char)(0x80 | ((cp >> 12) & 0x3F));
      o += (char)(0x80 | ((cp >> 6) & 0x3F));
      o += (char)(0x80 | (cp & 0x3F));
    }
  }
  bool hex4(uint32_t& v) {
    if (end - p < 4) return false;
    v = 0;
    for (int i = 0; i < 4; i++) {
      const char c = *p++;
      v <<= 4;
      if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
      else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
      else return false;
    }
    return true;
  }
  bool string(std::string& o) {
    if (p >= end || *p != '"') return false;
    p++;
    while (p < end && *p != '"') {
      const unsigned char c = (unsigned char)*p++;
      if (c < 0x20) return false;
      if (c != '\\') {
        o += (char)c;
        continue;
      }
      if (p >= end) return false;
      const char e = *p++;
      switch (e) {
        case '"': o += '"'; break;
        case '\\': o += '\\'; break;
        case '/': o += '/'; break;
        case 'b': o += '\b'; break;
        case 'f': o += '\f'; break;
        case 'n': o += '\n'; break;
        case 'r': o += '\r'; break;
        case 't': o += '\t'; break;
        case 'u': {
          uint32_t cp;
          if (!hex4(cp)) return false;
          if (cp >= 0xD800 && cp < 0xDC00) {  // surrogate pair
            uint32_t lo;
            if (end - p < 2 || p[0] != '\\' || p[1] != 'u') return false;
            p += 2;
            if (!hex4(lo) || lo < 0xDC00 || lo >= 0xE000) return false;
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          utf8(o, cp);
          break;
        }
        default: return false;
      }
    }
    if (p >= end) return false;
    p++;
    return true;
  }
  bool number(double& v) {
    const char* s = p;
    if (p < end && *p == '-') p++;
    if (p >= end || !(*p >= '0' && *p <= '9')) return false;
    while (p < end && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' || *p == '+' || *p == '-'))
      p++;
    const std::string t(s, p);
    char* e = nullptr;
    v = strtod(t.c_str(), &e);
    return e && *e == 0;
  }
  bool value(Json& j) {
    if (++depth > 64) return false;
    ws();
    bool ok = false;
    if (p >= end) {
      ok = false;
    } else if (*p == '{') {
      p++;
      j.kind = Json::Obj;
      ws();
      if (p < end && *p == '}') {
        p++;
        ok = true;
      } else {
        for (;;) {
          ws();
          std::string k;
          Json v;
          if (!string(k)) break;
          ws();
          if (p >= end || *p != ':') break;
          p++;
          if (!value(v)) break;
          j.obj.emplace_back(std::move(k), std::move(v));
          ws();
          if (p < end && *p == ',') {
            p++;
            continue;
          }
          if (p < end && *p == '}') {
            p++;
            ok = true;
          }
          break;
        }
      }
    } else if (*p == '[') {
      p++;
      j.kind = Json::Arr;
      ws();
      if (p < end && *p == ']') {
        p++;
        ok = true;
      } else {
        for (;;) {
          Json v;
          if (!value(v)) break;
          j.arr.push_back(std::move(v));
          ws();
          if (p < end && *p == ',') {
            p++;
            continue;
          }
          if (p < end && *p == ']') {
            p++;
            ok = true;
          }
          break;
        }
      }
    } else if (*p == '"') {
      j.kind = Json::Str;
      ok = string(j.str);
    } else if (lit("true")) {
      j.kind = Json::Bool;
      j.b = true;
      ok = true;
    } else if (lit("false")) {
      j.kind = Json::Bool;
      ok = true;
    } else if (lit("null")) {
      j.kind = Json::Null;
      ok = true;
    } else {
      j.kind = Json::Num;
      ok = number(j.num);
    }
    depth--;
    return ok;
  }
};

bool parse_json(const char* s, size_t n, Json& out) {
  JsonParser jp{s, s + n};
  // a UTF-8 byte order mark is accepted, as System.Text.Json does
  if (n >= 3 && (unsigned char)s[0] == 0xEF && (unsigned char)s[1] == 0xBB && (unsigned char)s[2] == 0xBF) jp.p += 3;
  if (!jp.value(out)) return false;
  jp.ws();
  return jp.p == jp.end;
}

// ------------------------------------------------------------- the reader --
struct CkptHeader {
  int vocab = 0, ctx = 0, d = 0, layers = 0, heads = 0;
  std::string name, arch;
  std::vector<std::string> names;
  bool has_training = false, has_moments = false;
};

namespace {

constexpr char kMagic[] = "FORGEMODEL1";
constexpr int kMagicLen = 11;
constexpr int kChecksum = 32;
constexpr char kArch[] = "forge-gpt2-tied-v1";

// reads exactly n bytes through the hash, within the content region
struct Reader {
  FILE* f;
  Sha256 sha;
  int64_t pos = 0, content = 0;
  bool read(void* dst, size_t n) {
    if (pos + (int64_t)n > content) return false;
    if (fread(dst, 1, n, f) != n) return false;
    sha.update(dst, n);
    pos += (int64_t)n;
    return true;
  }
};

bool json_int(const Json* j, int& v) {
  if (!j || j->kind != Json::Num || j->num != (double)(int)j->num) return false;
  v = (int)j->num;
  return true;
}

}  // namespace

// Validates `path` as Checkpoint.LoadCore does.  The registry check and the
// payload size need the model's names and parameter count, which depend on the
// header: `registry(hdr, &names, &nparams)` supplies them (returns "" or a
// model-configuration message).  With `weights` the weight payload is returned
// (registry order); the optimizer moments, when present, are hashed and dropped.
// With `header_only` it stops after the header, names and payload-size checks.
// Returns "" on success, else the reference's exception message; *data_error
// tells an InvalidDataException from a configuration error.
std::string read_checkpoint(const char* path, CkptHeader* hdr,
                            std::string (*registry)(const CkptHeader&, std::vector<std::string>*, int64_t*),
                            std::vector<float>* weights, bool header_only, bool* data_error) {
  *data_error = true;
  FILE* f = fopen(path, "rb");
  if (!f) {
    *data_error = false;
    return std::string("Could not find file '") + path + "'.";
  }
  struct Closer {
    FILE* f;
    ~Closer() { fclose(f); }
  } closer{f};
  if (fseeko(f, 0, SEEK_END) != 0) return "Unable to read the checkpoint.";
  const int64_t flen = ftello(f);
  fseeko(f, 0, SEEK_SET);
  char magic[kMagicLen];
  if (flen < kMagicLen || fread(magic, 1, kMagicLen, f) != (size_t)kMagicLen)
    return "Unable to read beyond the end of the stream.";
  if (memcmp(magic, kMagic, kMagicLen) != 0)
    return std::string("'") + path + "' is not a current FORGEMODEL1 checkpoint.";
  Reader r{f};
  r.content = flen - kChecksum;
  if (r.content < kMagicLen) return "Checkpoint is too short to contain its checksum.";
  r.sha.update(magic, kMagicLen);
  r.pos = kMagicLen;

  uint8_t lb[4];
  if (!r.read(lb, 4)) return "Unable to read beyond the end of the stream.";
  const int32_t jlen = (int32_t)((uint32_t)lb[0] | (uint32_t)lb[1] << 8 | (uint32_t)lb[2] << 16 | (uint32_t)lb[3] << 24);
  if (jlen <= 0 || jlen > (1 << 20)) return "Implausible header length " + std::to_string(jlen) + ".";
  std::string json((size_t)jlen, '\0');
  if (!r.read(&json[0], (size_t)jlen)) return "Checkpoint ended inside its JSON header.";
  Json h;
  if (!parse_json(json.data(), json.size(), h) || h.kind != Json::Obj) return "Checkpoint header failed to parse.";
  // properties the JSON omits keep the Header class defaults (0, "", [], null)
  const Json* a = h.get("Architecture");
  const Json* mn = h.get("ModelName");
  const Json* names = h.get("Names");
  const Json* tr = h.get("Training");
  const char* ikeys[5] = {"VocabSize", "ContextLength", "DModel", "NLayers", "NHeads"};
  int* ivals[5] = {&hdr->vocab, &hdr->ctx, &hdr->d, &hdr->layers, &hdr->heads};
  for (int i = 0; i < 5; i++) {
    const Json* v = h.get(ikeys[i]);
    if (v && v->kind != Json::Null && !json_int(v, *ivals[i])) return "Checkpoint header failed to parse.";
  }
  if (a && a->kind == Json::Str) hdr->arch = a->str;
  else if (a && a->kind != Json::Null) return "Checkpoint header failed to parse.";
  if (mn && mn->kind == Json::Str) hdr->name = mn->str;
  else if (mn && mn->kind != Json::Null) return "Checkpoint header failed to parse.";
  if (names && names->kind == Json::Arr) {
    for (auto& e : names->arr) {
      if (e.kind != Json::Str) return "Checkpoint header failed to parse.";
      hdr->names.push_back(e.str);
    }
  } else if (names && names->kind != Json::Null) {
    return "Checkpoint header failed to parse.";
  }
  hdr->has_training = tr && tr->kind == Json::Obj;
  if (tr && !hdr->has_training && tr->kind != Json::Null) return "Checkpoint header failed to parse.";
  if (hdr->has_training) {
    const Json* hm = tr->get("HasOptimizerState");
    if (hm && hm->kind == Json::Bool) hdr->has_moments = hm->b;
    else if (hm && hm->kind != Json::Null) return "Checkpoint header failed to parse.";
  }
  if (hdr->arch != kArch) return "Unsupported checkpoint architecture '" + hdr->arch + "'.";
  bool blank = true;
  for (char c : hdr->name)
    if (!(c == ' ' || c == '\t' || c == '\n' || c == '\r' || c == '\v' || c == '\f')) blank = false;
  if (blank) return "Checkpoint is missing its Forge model name.";
  if (!hdr->has_training) return "Training checkpoint is missing its training-state header.";

  std::vector<std::string> reg;
  int64_t nparams = 0;
  const std::string cfg = registry(*hdr, &reg, &nparams);
  if (!cfg.empty()) {
    *data_error = false;  // ModelConfig's own ArgumentException
    return cfg;
  }
  if (hdr->names != reg) return "Checkpoint parameter names do not match the model registry.";
  const int64_t wbytes = nparams * 4;
  const int64_t expected = wbytes * (hdr->has_moments ? 3 : 1);
  if (r.content - r.pos != expected)
    return "Checkpoint payload is " + std::to_string(r.content - r.pos) + " bytes, expected " +
           std::to_string(expected) + ".";
  if (header_only) return "";
  if (weights) {
    weights->resize((size_t)nparams);
    // little-endian fp32 on a little-endian host: the bytes are the floats
    if (!r.read(weights->data(), (size_t)wbytes)) return "Unable to read beyond the end of the stream.";
  }
  std::vector<char> buf(1 << 20);
  while (r.pos < r.content) {
    const size_t n = (size_t)std::min<int64_t>((int64_t)buf.size(), r.content - r.pos);
    if (!r.read(buf.data(), n)) return "Unable to read beyond the end of the stream.";
  }
  uint8_t want[kChecksum], got[kChecksum];
  if (fread(want, 1, kChecksum, f) != (size_t)kChecksum) return "Unable to read beyond the end of the stream.";
  r.sha.final(got);
  if (memcmp(want, got, kChecksum) != 0) return "Checkpoint SHA-256 checksum does not match; the file is corrupted.";
  return "";
}

}  // namespace fh
