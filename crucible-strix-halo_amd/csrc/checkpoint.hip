// Safetensors checkpoints on the host and the EXL3 linear loader.
//
// A checkpoint is one .safetensors file or a directory whose
// model.safetensors.index.json maps tensor names to shard files (the reference's
// st::Checkpoint, engine/exl3/safetensors.h).  Every shard is memory-mapped read-only
// when the checkpoint opens; its header (8-byte little-endian length, then a JSON object
// of {name: {dtype, shape, data_offsets}}) is parsed by a bounded recursive-descent
// reader and every tensor is checked: known dtype, non-negative shape, offsets inside
// the payload, shape x dtype bytes == offset span, unique names.
//
// The EXL3 loader validates one linear's tensors (docs/EXL3_FORMAT.md §2 of the
// reference: prefix.trellis I16 [I/16][O/16][8 k2], prefix.suh F16 [I], prefix.svh F16
// [O], codebook marker prefix.mul1 = 0x83DCD12D or prefix.mcg = 0xCBAC1FED as I32
// scalars, neither = 3inst) and uploads it into caller-owned device buffers, repacking
// the trellis on the device (engine/model/flashnext/model.h:503-527).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdio>
#include <cstring>
#include <fstream>
#include <iterator>
#include <map>
#include <new>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "internal.hpp"

namespace cx {
namespace {

thread_local std::string g_error;

int SetError(int rc, const std::string& msg) {
  g_error = msg;
  return rc;
}

struct Tensor {
  int dtype = -1;
  std::vector<int64_t> shape;
  const uint8_t* data = nullptr;
  uint64_t bytes = 0;
};

struct Shard {
  const uint8_t* base = nullptr;
  size_t size = 0;
};

// dtype name -> (code, element bytes)
bool DtypeOf(const std::string& s, int* code, int* bytes) {
  static const std::pair<const char*, std::pair<int, int>> kTable[] = {
      {"BOOL", {CX_DT_BOOL, 1}}, {"U8", {CX_DT_U8, 1}},   {"I8", {CX_DT_I8, 1}},     {"I16", {CX_DT_I16, 2}},
      {"U16", {CX_DT_U16, 2}},   {"F16", {CX_DT_F16, 2}}, {"BF16", {CX_DT_BF16, 2}}, {"I32", {CX_DT_I32, 4}},
      {"U32", {CX_DT_U32, 4}},   {"F32", {CX_DT_F32, 4}}, {"I64", {CX_DT_I64, 8}},   {"U64", {CX_DT_U64, 8}},
      {"F64", {CX_DT_F64, 8}},
  };
  for (const auto& e : kTable)
    if (s == e.first) {
      *code = e.second.first;
      *bytes = e.second.second;
      return true;
    }
  return false;
}

// Bounded JSON reader over one buffer.  Errors throw a message with the byte position.
class Json {
 public:
  explicit Json(const char* p, size_t n) : p_(p), n_(n) {}
  void Fail(const std::string& what) const { throw std::runtime_error(what + " at JSON byte " + std::to_string(i_)); }
  void Space() {
    while (i_ < n_ && (p_[i_] == ' ' || p_[i_] == '\t' || p_[i_] == '\n' || p_[i_] == '\r')) ++i_;
  }
  bool At(char c) {
    Space();
    return i_ < n_ && p_[i_] == c;
  }
  void Eat(char c) {
    if (!At(c)) Fail(std::string("expected '") + c + "'");
    ++i_;
  }
  // After a member or element: ',' then more (no trailing comma), or the closer.
  bool More(char close) {
    if (At(close)) {
      ++i_;
      return false;
    }
    Eat(',');
    if (At(close)) Fail("trailing comma");
    return true;
  }
  std::string String() {
    Eat('"');
    std::string out;
    for (;;) {
      if (i_ >= n_) Fail("unterminated string");
      const unsigned char c = (unsigned char)p_[i_++];
      if (c == '"') return out;
      if (c < 0x20) Fail("control character in string");
      if (c != '\\') {
        out += (char)c;
        continue;
      }
      if (i_ >= n_) Fail("unterminated escape");
      const char e = p_[i_++];
      switch (e) {
        case '"': case '\\': case '/': out += e; break;
        case 'b': out += '\b'; break;
        case 'f': out += '\f'; break;
        case 'n': out += '\n'; break;
        case 'r': out += '\r'; break;
        case 't': out += '\t'; break;
        case 'u': Utf8(out, CodePoint()); break;
        default: Fail("invalid escape");
      }
    }
  }
  int64_t Integer() {
    Space();
    const size_t s = i_;
    bool neg = false;
    if (i_ < n_ && p_[i_] == '-') neg = true, ++i_;
    if (i_ >= n_ || p_[i_] < '0' || p_[i_] > '9') Fail("expected integer");
    if (p_[i_] == '0' && i_ + 1 < n_ && p_[i_ + 1] >= '0' && p_[i_ + 1] <= '9') Fail("leading zero");
    uint64_t v = 0;
    while (i_ < n_ && p_[i_] >= '0' && p_[i_] <= '9') {
      const uint64_t d = (uint64_t)(p_[i_++] - '0');
      if (v > (uint64_t(INT64_MAX) - d) / 10) Fail("integer overflow");
      v = v * 10 + d;
    }
    if (i_ < n_ && (p_[i_] == '.' || p_[i_] == 'e' || p_[i_] == 'E')) {
      i_ = s;
      Fail("expected an integer, got a fraction");
    }
    return neg ? -(int64_t)v : (int64_t)v;
  }
  std::vector<int64_t> Integers() {
    std::vector<int64_t> v;
    Eat('[');
    if (At(']')) {
      ++i_;
      return v;
    }
    do v.push_back(Integer());
    while (More(']'));
    return v;
  }
  void Skip(int depth = 0) {
    if (depth > 64) Fail("nesting deeper than 64");
    Space();
    if (i_ >= n_) Fail("missing value");
    const char c = p_[i_];
    if (c == '"') {
      String();
    } else if (c == '{' || c == '[') {
      const char close = c == '{' ? '}' : ']';
      ++i_;
      if (At(close)) {
        ++i_;
        return;
      }
      do {
        if (c == '{') {
          String();
          Eat(':');
        }
        Skip(depth + 1);
      } while (More(close));
    } else if (c == 't' || c == 'f' || c == 'n') {
      const char* lit = c == 't' ? "true" : c == 'f' ? "false" : "null";
      const size_t L = std::strlen(lit);
      if (n_ - i_ < L || std::memcmp(p_ + i_, lit, L)) Fail("invalid literal");
      i_ += L;
    } else {
      Number();
    }
  }
  void End() {
    Space();
    if (i_ != n_) Fail("trailing data after the JSON object");
  }

 private:
  void Number() {
    if (i_ < n_ && p_[i_] == '-') ++i_;
    Digits();
    if (i_ < n_ && p_[i_] == '.') ++i_, Digits();
    if (i_ < n_ && (p_[i_] == 'e' || p_[i_] == 'E')) {
      ++i_;
      if (i_ < n_ && (p_[i_] == '+' || p_[i_] == '-')) ++i_;
      Digits();
    }
  }
  void Digits() {
    if (i_ >= n_ || p_[i_] < '0' || p_[i_] > '9') Fail("expected digit");
    while (i_ < n_ && p_[i_] >= '0' && p_[i_] <= '9') ++i_;
  }
  uint32_t Hex4() {
    if (n_ - i_ < 4) Fail("short \\u escape");
    uint32_t v = 0;
    for (int k = 0; k < 4; ++k) {
      const char c = p_[i_++];
      int d = c >= '0' && c <= '9' ? c - '0' : c >= 'a' && c <= 'f' ? c - 'a' + 10 : c >= 'A' && c <= 'F' ? c - 'A' + 10 : -1;
      if (d < 0) Fail("bad hex digit");
      v = v * 16 + (uint32_t)d;
    }
    return v;
  }
  uint32_t CodePoint() {
    uint32_t u = Hex4();
    if (u >= 0xD800 && u < 0xDC00) {
      if (n_ - i_ < 2 || p_[i_] != '\\' || p_[i_ + 1] != 'u') Fail("lone high surrogate");
      i_ += 2;
      const uint32_t lo = Hex4();
      if (lo < 0xDC00 || lo > 0xDFFF) Fail("bad low surrogate");
      u = 0x10000 + ((u - 0xD800) << 10) + (lo - 0xDC00);
    } else if (u >= 0xDC00 && u <= 0xDFFF) {
      Fail("lone low surrogate");
    }
    return u;
  }
  static void Utf8(std::string& out, uint32_t u) {
    if (u < 0x80) {
      out += (char)u;
    } else if (u < 0x800) {
      out += (char)(0xC0 | (u >> 6));
      out += (char)(0x80 | (u & 63));
    } else if (u < 0x10000) {
      out += (char)(0xE0 | (u >> 12));
      out += (char)(0x80 | ((u >> 6) & 63));
      out += (char)(0x80 | (u & 63));
    } else {
      out += (char)(0xF0 | (u >> 18));
      out += (char)(0x80 | ((u >> 12) & 63));
      out += (char)(0x80 | ((u >> 6) & 63));
      out += (char)(0x80 | (u & 63));
    }
  }
  const char* p_;
  size_t n_, i_ = 0;
};

std::string BaseName(const std::string& path) { return path.substr(path.find_last_of('/') + 1); }

}  // namespace
}  // namespace cx

struct cx_checkpoint {
  std::vector<cx::Shard> shards;
  std::map<std::string, cx::Tensor> tensors;
};

namespace cx {
namespace {

// Maps one shard and adds its tensors.  Throws on any format error.
void LoadShard(cx_checkpoint* ck, const std::string& path, const std::map<std::string, std::string>* owner) {
  const int fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0) throw std::runtime_error("cannot open " + BaseName(path) + ": " + std::strerror(errno));
  struct stat sb {};
  if (fstat(fd, &sb) != 0 || !S_ISREG(sb.st_mode) || sb.st_size < 8) {
    close(fd);
    throw std::runtime_error(BaseName(path) + ": not a regular file of at least 8 bytes");
  }
  void* p = mmap(nullptr, (size_t)sb.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  if (p == MAP_FAILED) throw std::runtime_error(BaseName(path) + ": mmap failed");
  const Shard sh{static_cast<const uint8_t*>(p), (size_t)sb.st_size};
  ck->shards.push_back(sh);
  uint64_t hlen = 0;
  for (int b = 0; b < 8; ++b) hlen |= (uint64_t)sh.base[b] << (8 * b);
  if (hlen > sh.size - 8) throw std::runtime_error(BaseName(path) + ": header length exceeds the file");
  const uint64_t data0 = 8 + hlen, payload = sh.size - data0;
  Json js(reinterpret_cast<const char*>(sh.base + 8), (size_t)hlen);
  std::string name;
  try {
    js.Eat('{');
    if (js.At('}')) {
      js.Eat('}');
    } else {
      do {
        name = js.String();
        js.Eat(':');
        if (name == "__metadata__") {
          js.Skip();
          continue;
        }
        Tensor t;
        std::string dtype;
        std::vector<int64_t> off;
        unsigned seen = 0;
        js.Eat('{');
        if (!js.At('}')) {
          do {
            const std::string key = js.String();
            js.Eat(':');
            const unsigned bit = key == "dtype" ? 1u : key == "shape" ? 2u : key == "data_offsets" ? 4u : 0u;
            if (bit & seen) throw std::runtime_error("duplicate field " + key);
            seen |= bit;
            if (bit == 1) dtype = js.String();
            else if (bit == 2) t.shape = js.Integers();
            else if (bit == 4) off = js.Integers();
            else js.Skip(1);
          } while (js.More('}'));
        } else {
          js.Eat('}');
        }
        if (seen != 7) throw std::runtime_error("missing dtype, shape or data_offsets");
        int esz = 0;
        if (!DtypeOf(dtype, &t.dtype, &esz)) throw std::runtime_error("unsupported dtype " + dtype);
        if (off.size() != 2 || off[0] < 0 || off[1] < off[0] || (uint64_t)off[1] > payload)
          throw std::runtime_error("data_offsets outside the payload");
        unsigned __int128 bytes = (unsigned)esz;
        for (const int64_t d : t.shape) {
          if (d < 0) throw std::runtime_error("negative dimension");
          bytes *= (uint64_t)d;
          if (bytes > payload) throw std::runtime_error("shape larger than the payload");
        }
        if ((uint64_t)bytes != (uint64_t)(off[1] - off[0]))
          throw std::runtime_error("shape and dtype do not match the data_offsets span");
        t.data = sh.base + data0 + off[0];
        t.bytes = (uint64_t)bytes;
        if (owner) {  // sharded: only the names the index gives to this file
          const auto it = owner->find(name);
          if (it == owner->end() || BaseName(path) != it->second) continue;
        }
        if (!ck->tensors.emplace(name, t).second) throw std::runtime_error("duplicate tensor name");
      } while (js.More('}'));
    }
    js.End();
  } catch (const std::runtime_error& e) {
    throw std::runtime_error(BaseName(path) + (name.empty() ? "" : ", tensor " + name) + ": " + e.what());
  }
}

const Tensor* Find(const cx_checkpoint* ck, const std::string& name) {
  const auto it = ck->tensors.find(name);
  return it == ck->tensors.end() ? nullptr : &it->second;
}

}  // namespace
}  // namespace cx

using namespace cx;

extern "C" {

const char* cx_last_error(void) { return g_error.c_str(); }

int cx_checkpoint_open(const char* path, cx_checkpoint** out) {
  if (!path || !out) return SetError(CX_E_ARG, "null argument");
  *out = nullptr;
  auto* ck = new (std::nothrow) cx_checkpoint();
  if (!ck) return SetError(CX_E_ARG, "out of host memory");
  try {
    struct stat sb {};
    if (stat(path, &sb) != 0) throw std::runtime_error(std::string("cannot open ") + BaseName(path));
    if (S_ISDIR(sb.st_mode)) {
      const std::string dir(path), index = dir + "/model.safetensors.index.json";
      std::ifstream f(index, std::ios::binary);
      if (!f) throw std::runtime_error("cannot open model.safetensors.index.json");
      std::stringstream ss;
      ss << f.rdbuf();
      const std::string s = ss.str();
      std::map<std::string, std::string> owner;
      std::vector<std::string> files;
      Json js(s.data(), s.size());
      bool have_map = false;
      try {
        js.Eat('{');
        if (!js.At('}')) {
          do {
            const std::string key = js.String();
            js.Eat(':');
            if (key != "weight_map") {
              js.Skip();
              continue;
            }
            if (have_map) throw std::runtime_error("duplicate weight_map");
            have_map = true;
            js.Eat('{');
            if (js.At('}')) {
              js.Eat('}');
              continue;
            }
            do {
              const std::string name = js.String();
              js.Eat(':');
              const std::string file = js.String();
              if (file.empty() || file == "." || file == ".." || file.find('/') != std::string::npos ||
                  file.find('\\') != std::string::npos || file.find('\0') != std::string::npos)
                throw std::runtime_error("shard name must be a plain file name");
              if (!owner.emplace(name, file).second) throw std::runtime_error("duplicate index entry " + name);
              bool known = false;
              for (const auto& x : files) known |= x == file;
              if (!known) files.push_back(file);
            } while (js.More('}'));
          } while (js.More('}'));
        } else {
          js.Eat('}');
        }
        js.End();
      } catch (const std::runtime_error& e) {
        throw std::runtime_error(std::string("model.safetensors.index.json: ") + e.what());
      }
      if (!have_map) throw std::runtime_error("model.safetensors.index.json: missing weight_map");
      for (const auto& file : files) LoadShard(ck, dir + "/" + file, &owner);
      for (const auto& [name, file] : owner)
        if (!ck->tensors.count(name)) throw std::runtime_error(file + ", tensor " + name + ": missing from its shard");
    } else {
      LoadShard(ck, path, nullptr);
    }
  } catch (const std::runtime_error& e) {
    cx_checkpoint_close(ck);
    return SetError(CX_E_FORMAT, e.what());
  }
  *out = ck;
  g_error.clear();
  return CX_OK;
}

void cx_checkpoint_close(cx_checkpoint* ck) {
  if (!ck) return;
  for (const auto& sh : ck->shards) munmap(const_cast<uint8_t*>(sh.base), sh.size);
  delete ck;
}

int32_t cx_checkpoint_count(const cx_checkpoint* ck) { return ck ? (int32_t)ck->tensors.size() : 0; }

const char* cx_checkpoint_name(const cx_checkpoint* ck, int32_t i) {
  if (!ck || i < 0 || i >= (int32_t)ck->tensors.size()) return nullptr;
  auto it = ck->tensors.begin();
  std::advance(it, i);
  return it->first.c_str();
}

int cx_checkpoint_tensor(const cx_checkpoint* ck, const char* name, int32_t* dtype, int32_t* rank, int64_t* shape,
                         const void** data, uint64_t* bytes) {
  if (!ck || !name) return SetError(CX_E_ARG, "null argument");
  const Tensor* t = Find(ck, name);
  if (!t) return SetError(CX_E_FORMAT, std::string("tensor ") + name + ": not in the checkpoint");
  if (t->shape.size() > CX_MAX_RANK) return SetError(CX_E_FORMAT, std::string("tensor ") + name + ": rank above 8");
  if (dtype) *dtype = t->dtype;
  if (rank) *rank = (int32_t)t->shape.size();
  if (shape)
    for (size_t d = 0; d < t->shape.size(); ++d) shape[d] = t->shape[d];
  if (data) *data = t->data;
  if (bytes) *bytes = t->bytes;
  return CX_OK;
}

int cx_exl3_linear_info(const cx_checkpoint* ck, const char* prefix, int32_t* in_features, int32_t* out_features,
                        int32_t* k2, int32_t* codebook) {
  if (!ck || !prefix) return SetError(CX_E_ARG, "null argument");
  const std::string p(prefix);
  auto fail = [&](const std::string& why) { return SetError(CX_E_FORMAT, "linear " + p + ": " + why); };
  const Tensor* tr = Find(ck, p + ".trellis");
  if (!tr) return fail("missing .trellis");
  if (tr->dtype != CX_DT_I16 || tr->shape.size() != 3) return fail(".trellis must be I16 [I/16][O/16][8 k2]");
  const int64_t A = tr->shape[0], B = tr->shape[1], W = tr->shape[2];
  if (W % 8 || !ValidK2((int)(W / 8))) return fail(".trellis last dimension is not 16 K for a supported K");
  if (A <= 0 || B <= 0 || A % 8 || B % 8 || A * 16 > (1 << 30) || B * 16 > (1 << 30))
    return fail("in and out features must be positive multiples of 128");
  const int I = (int)(A * 16), O = (int)(B * 16);
  const Tensor* suh = Find(ck, p + ".suh");
  const Tensor* svh = Find(ck, p + ".svh");
  if (!suh || suh->dtype != CX_DT_F16 || suh->shape != std::vector<int64_t>{I}) return fail(".suh must be F16 [I]");
  if (!svh || svh->dtype != CX_DT_F16 || svh->shape != std::vector<int64_t>{O}) return fail(".svh must be F16 [O]");
  auto marker = [&](const char* suffix, uint32_t expect, bool* present) -> int {
    const Tensor* m = Find(ck, p + suffix);
    *present = m != nullptr;
    if (!m) return CX_OK;
    if (m->dtype != CX_DT_I32 || !m->shape.empty()) return fail(std::string(suffix) + " must be an I32 scalar");
    uint32_t v;
    std::memcpy(&v, m->data, 4);
    if (v != expect) return fail(std::string(suffix) + " holds an unknown multiplier");
    return CX_OK;
  };
  bool mul1 = false, mcg = false;
  int rc;
  if ((rc = marker(".mul1", 0x83DCD12Du, &mul1)) || (rc = marker(".mcg", 0xCBAC1FEDu, &mcg))) return rc;
  if (mul1 && mcg) return fail("both .mul1 and .mcg markers");
  const int cb = mul1 ? CX_CB_MUL1 : mcg ? CX_CB_MCG : CX_CB_3INST;
  const int kk = (int)(W / 8);
  if (cb != CX_CB_MUL1 && (kk & 1)) return fail("mcg / 3inst need a whole number of bits per weight");
  if (in_features) *in_features = I;
  if (out_features) *out_features = O;
  if (k2) *k2 = kk;
  if (codebook) *codebook = cb;
  return CX_OK;
}

int cx_exl3_load_linear(const cx_checkpoint* ck, const char* prefix, cx_exl3_matrix* m, uint32_t* tiles,
                        uint16_t* suh, uint16_t* svh, void* staging, size_t staging_bytes, cx_stream_t stream) {
  if (!m || !tiles || !suh || !svh || !staging) return SetError(CX_E_ARG, "null argument");
  int32_t I, O, k2, cb;
  int rc = cx_exl3_linear_info(ck, prefix, &I, &O, &k2, &cb);
  if (rc) return rc;
  const std::string p(prefix);
  const Tensor* tr = Find(ck, p + ".trellis");
  if (staging_bytes < tr->bytes) return SetError(CX_E_WORKSPACE, "staging buffer smaller than the trellis");
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  if ((e = hipMemcpyAsync(staging, tr->data, tr->bytes, hipMemcpyHostToDevice, s)) != hipSuccess ||
      (e = hipMemcpyAsync(suh, Find(ck, p + ".suh")->data, (size_t)I * 2, hipMemcpyHostToDevice, s)) != hipSuccess ||
      (e = hipMemcpyAsync(svh, Find(ck, p + ".svh")->data, (size_t)O * 2, hipMemcpyHostToDevice, s)) != hipSuccess)
    return SetError((int)e, "upload failed");
  if ((rc = cx_exl3_repack(static_cast<const int16_t*>(staging), I, O, k2, tiles, stream))) return rc;
  // The copies read pageable host memory the mapping owns; finish them before returning
  // so the caller may close the checkpoint.
  if ((e = hipStreamSynchronize(s)) != hipSuccess) return SetError((int)e, "synchronize failed");
  *m = cx_exl3_matrix{tiles, suh, svh, I, O, k2, cb};
  return CX_OK;
}

}  // extern "C"
