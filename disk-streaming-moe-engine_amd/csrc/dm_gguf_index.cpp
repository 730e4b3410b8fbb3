// dm_gguf_index.cpp -- the GGUF container index of src/format/gguf.mojo:144-411 and
// the payload read of stream_gguf_tensor_f32 (gguf.mojo:563-596), on the host.
//
// Integer arithmetic follows the reference's signed 64-bit Int: products and
// sums wrap, and `//` floors.  Error texts are the reference's.
#include <stdio.h>

#include <string>
#include <vector>

#include "dm_gguf.h"
#include "dm_formats.h"

namespace dm {
namespace {

struct Fail {
  std::string msg;
};
[[noreturn]] void fail(std::string m) { throw Fail{std::move(m)}; }

int64_t wadd(int64_t a, int64_t b) { return (int64_t)((uint64_t)a + (uint64_t)b); }
int64_t wmul(int64_t a, int64_t b) { return (int64_t)((uint64_t)a * (uint64_t)b); }
int64_t fdiv(int64_t a, int64_t b) {  // floor division, b > 0
  const int64_t q = a / b;
  return (a % b != 0 && a < 0) ? q - 1 : q;
}

struct Fh {
  FILE* f = nullptr;
  ~Fh() {
    if (f) fclose(f);
  }
};

// Little-endian cursor over the first bytes of the file (ByteReader,
// gguf.mojo:144-215).
class Cursor {
 public:
  explicit Cursor(std::vector<uint8_t> b) : b_(std::move(b)) {}
  int64_t pos = 0;

  bool have(int64_t n) const { return pos + n <= (int64_t)b_.size(); }
  int64_t u8() {
    if (!have(1)) fail("GGUF: unexpected EOF reading u8");
    return b_[pos++];
  }
  int64_t u16() {
    if (!have(2)) fail("GGUF: unexpected EOF reading u16");
    const int64_t v = b_[pos] | (b_[pos + 1] << 8);
    pos += 2;
    return v;
  }
  int64_t u32() {
    if (!have(4)) fail("GGUF: unexpected EOF reading u32");
    int64_t v = 0;
    for (int i = 3; i >= 0; --i) v = (v << 8) | b_[pos + i];
    pos += 4;
    return v;
  }
  // values with the top bit set are rejected: the reference keeps them in a
  // signed Int
  int64_t u64() {
    if (!have(8)) fail("GGUF_FILE_CORRUPT: unexpected EOF reading u64");
    if (b_[pos + 7] & 0x80) fail("GGUF_FILE_CORRUPT: u64 overflow/negative value");
    int64_t v = 0;
    for (int i = 7; i >= 0; --i) v = (v << 8) | b_[pos + i];
    pos += 8;
    return v;
  }
  std::string str() {
    const int64_t n = u64();
    if (n > 65536) fail("GGUF: string length invalid: " + std::to_string(n));
    if (!have(n)) fail("GGUF: unexpected EOF reading string");
    std::string s(reinterpret_cast<const char*>(b_.data() + pos), (size_t)n);
    pos += n;
    return s;
  }

 private:
  std::vector<uint8_t> b_;
};

// One metadata value (_skip_gguf_value, gguf.mojo:218-254): its text for
// scalars and strings, "[Array of N elements]" for arrays.  Nested arrays
// are walked with an explicit stack.
std::string read_value(Cursor& c, int64_t vtype) {
  struct Level {
    int64_t type, left;
  };
  std::vector<Level> stack;
  std::string top;
  for (;;) {
    std::string v;
    switch (vtype) {
      case 0: case 1: case 7: v = std::to_string(c.u8()); break;    // u8, i8, bool
      case 2: case 3: v = std::to_string(c.u16()); break;           // u16, i16
      case 4: case 5: case 6: v = std::to_string(c.u32()); break;   // u32, i32, f32 bits
      case 10: case 11: case 12: v = std::to_string(c.u64()); break;  // u64, i64, f64 bits
      case 8: v = c.str(); break;
      case 9: {
        const int64_t et = c.u32();
        const int64_t n = c.u64();
        v = "[Array of " + std::to_string(n) + " elements]";
        if (stack.empty()) top = v;
        stack.push_back({et, n});
        break;
      }
      default: fail("GGUF: unknown value type " + std::to_string(vtype));
    }
    if (stack.empty()) return v;
    while (!stack.empty() && stack.back().left == 0) stack.pop_back();
    if (stack.empty()) return top;
    --stack.back().left;
    vtype = stack.back().type;
  }
}

// Int(val_str) of general.alignment (gguf.mojo:320-326): decimal with an
// optional sign; anything else leaves the alignment unchanged.
bool parse_int(const std::string& s, int64_t* v) {
  size_t i = 0, n = s.size();
  while (i < n && (s[i] == ' ' || s[i] == '\t')) ++i;
  while (n > i && (s[n - 1] == ' ' || s[n - 1] == '\t')) --n;
  bool neg = false;
  if (i < n && (s[i] == '+' || s[i] == '-')) neg = s[i++] == '-';
  if (i == n) return false;
  uint64_t a = 0;
  for (; i < n; ++i) {
    if (s[i] < '0' || s[i] > '9') return false;
    a = a * 10 + (uint64_t)(s[i] - '0');
    if (a > (uint64_t)INT64_MAX) return false;
  }
  *v = neg ? -(int64_t)a : (int64_t)a;
  return true;
}

// get_ggml_block_specs (gguf.mojo:76-102), with its (1, 4) fallback.
void block_spec_any(int64_t t, int64_t* bs, int64_t* bpb) {
  static const struct {
    int t, bs, bpb;
  } k[] = {{0, 1, 4},      {1, 1, 2},      {30, 1, 2},     {2, 32, 18},    {3, 32, 20},
           {8, 32, 34},    {11, 256, 114}, {12, 256, 144}, {13, 256, 176}, {14, 256, 210},
           {18, 256, 98},  {21, 256, 110}};
  *bs = 1;
  *bpb = 4;
  for (const auto& e : k)
    if (e.t == t) {
      *bs = e.bs;
      *bpb = e.bpb;
    }
}

}  // namespace

int GgufFile::find(const std::string& name) const {
  auto it = tensor_map.find(name);
  return it == tensor_map.end() ? -1 : it->second;
}

const std::string* GgufFile::meta(const std::string& key) const {
  auto it = meta_pos.find(key);
  return it == meta_pos.end() ? nullptr : &metadata[it->second].second;
}

bool parse_gguf_index(const std::string& path, GgufFile* out, std::string* err) {
  try {
    Fh fh;
    fh.f = fopen(path.c_str(), "rb");
    if (!fh.f) fail(error_json("FILE_NOT_FOUND", "tidak bisa open: " + path, path, ""));
    fseeko(fh.f, 0, SEEK_END);
    const int64_t filesize = (int64_t)ftello(fh.f);
    if (filesize < 32)
      fail("GGUF_FILE_CORRUPT: file size " + std::to_string(filesize) + " too small for header");
    // header and tensor directory are parsed from the first 4 MiB only
    std::vector<uint8_t> head((size_t)(filesize < (4 << 20) ? filesize : (4 << 20)));
    fseeko(fh.f, 0, SEEK_SET);
    if (fread(head.data(), 1, head.size(), fh.f) != head.size())
      fail("GGUF_FILE_CORRUPT: file size " + std::to_string(filesize) + " too small for header");
    Cursor c(std::move(head));
    static const uint8_t magic[4] = {'G', 'G', 'U', 'F'};
    for (int i = 0; i < 4; ++i)
      if (c.u8() != magic[i]) fail("GGUF_FILE_CORRUPT: invalid magic header (expected 'GGUF')");
    GgufFile g;
    g.path = path;
    g.filesize = filesize;
    g.version = (int)c.u32();
    if (g.version != 2 && g.version != 3)
      fail("GGUF_FILE_CORRUPT: unsupported version " + std::to_string(g.version));
    g.tensor_count = c.u64();
    g.metadata_kv_count = c.u64();
    if (g.tensor_count > 100000)
      fail("GGUF_FILE_CORRUPT: tensor_count out of bounds: " + std::to_string(g.tensor_count));

    for (int64_t k = 0; k < g.metadata_kv_count; ++k) {
      std::string key = c.str();
      const int64_t vt = c.u32();
      std::string val = read_value(c, vt);
      auto it = g.meta_pos.find(key);
      if (it == g.meta_pos.end()) {
        g.meta_pos.emplace(key, g.metadata.size());
        g.metadata.emplace_back(key, val);
      } else {
        g.metadata[it->second].second = val;
      }
      int64_t al = 0;
      if (key == "general.alignment" && parse_int(val, &al) && al > 0) g.alignment = al;
    }

    int64_t max_end = 0;
    for (int64_t i = 0; i < g.tensor_count; ++i) {
      GgufTensor t;
      t.name = c.str();
      const int64_t ndim = c.u32();
      if (ndim < 1 || ndim > 8)
        fail("GGUF_FILE_CORRUPT: tensor ndim invalid: " + std::to_string(ndim));
      int64_t ne = 1;
      for (int64_t d = 0; d < ndim; ++d) {
        t.dims.push_back(c.u64());
        ne = wmul(ne, t.dims.back());
      }
      t.type = (int)c.u32();
      t.offset = c.u64();
      int64_t bs, bpb;
      block_spec_any(t.type, &bs, &bpb);
      t.num_elements = ne;
      t.raw_bytes = wmul(fdiv(wadd(ne, bs - 1), bs), bpb);
      const int64_t end = wadd(t.offset, t.raw_bytes);
      if (end < t.offset) fail("GGUF_FILE_CORRUPT: tensor offset integer overflow");
      if (end > max_end) max_end = end;
      g.tensor_map[t.name] = (int)i;
      g.tensors.push_back(std::move(t));
    }
    g.data_section_offset = wmul(fdiv(wadd(c.pos, g.alignment - 1), g.alignment), g.alignment);
    for (const GgufTensor& t : g.tensors) {
      const int64_t end = wadd(wadd(g.data_section_offset, t.offset), t.raw_bytes);
      if (end > filesize || end < 0)
        fail("GGUF_FILE_CORRUPT: tensor extends beyond file boundary");
    }
    g.expected_file_size = wadd(g.data_section_offset, max_end);
    const int64_t diff = filesize - g.expected_file_size;
    if (diff != 0)
      fail("GGUF_FILE_CORRUPT: actual size " + std::to_string(filesize) + " != expected size " +
           std::to_string(g.expected_file_size) + " (diff: " + std::to_string(diff) + " bytes)");
    *out = std::move(g);
    return true;
  } catch (const Fail& f) {
    *err = f.msg;
    return false;
  }
}

bool read_gguf_tensor(const GgufFile& f, int idx, std::vector<uint8_t>* out, std::string* err) {
  const GgufTensor& t = f.tensors[(size_t)idx];
  Fh fh;
  fh.f = fopen(f.path.c_str(), "rb");
  if (!fh.f) {
    *err = error_json("FILE_NOT_FOUND", "tidak bisa open: " + f.path, f.path, "");
    return false;
  }
  out->resize((size_t)t.raw_bytes);
  size_t got = 0;
  if (fseeko(fh.f, (off_t)(f.data_section_offset + t.offset), SEEK_SET) == 0)
    got = fread(out->data(), 1, out->size(), fh.f);
  if ((int64_t)got < t.raw_bytes) {
    *err = "GGUF_READ_ERROR: truncated read for tensor " + t.name + ": expected " +
           std::to_string(t.raw_bytes) + " bytes, got " + std::to_string(got);
    return false;
  }
  return true;
}

}  // namespace dm
