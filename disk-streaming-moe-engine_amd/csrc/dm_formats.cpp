// dm_formats.cpp -- host readers of the reference's weight files.
//
// quant model (src/format/quant_reader.mojo): a 256-byte JSON header padded
// with spaces, then per tensor [u32 LE meta length][meta JSON][fp16 LE group
// scales][packed 4-bit codes], records back to back up to the end of the
// file.  safetensors (src/format/reader.mojo): [u64 LE header length][JSON
// header][payload], every tensor's [begin, end) inside the payload, the
// buffers tiling it without holes or overlap.
//
// Both JSON headers are read with a byte-level scanner that accepts the same
// subset as src/format/scanner.mojo (unsigned integers only, no fractions
// outside strings) and fails with the same error objects; the validation
// messages are those of the reference, so a caller sees identical text.
#include "dm_formats.h"

#include <stdio.h>

#include <algorithm>
#include <string>
#include <vector>

namespace dm {
namespace {

struct ParseFail {
  std::string msg;
};

std::string json_escape(const std::string& s) {  // types.mojo:15-49
  static const char* hex = "0123456789abcdef";
  std::string o;
  for (unsigned char b : s) {
    if (b == '"' || b == '\\') {
      o += '\\';
      o += (char)b;
    } else if (b == '\n') {
      o += "\\n";
    } else if (b == '\r') {
      o += "\\r";
    } else if (b == '\t') {
      o += "\\t";
    } else if (b == 8) {
      o += "\\b";
    } else if (b == 12) {
      o += "\\f";
    } else if (b < 32) {
      o += "\\u00";
      o += hex[b >> 4];
      o += hex[b & 15];
    } else {
      o += (char)b;
    }
  }
  return o;
}

std::string S(long long v) { return std::to_string(v); }

[[noreturn]] void fail(const std::string& type, const std::string& detail,
                       const std::string& shard, const std::string& tensor) {
  throw ParseFail{error_json(type, detail, shard, tensor)};
}

// The JSON subset scanner of src/format/scanner.mojo:11-352.
class Scanner {
 public:
  Scanner(const std::vector<uint8_t>& b, std::string shard) : buf_(b), shard_(std::move(shard)) {}
  size_t pos = 0;

  bool eof() const { return pos >= buf_.size(); }
  int peek() const { return eof() ? -1 : buf_[pos]; }

  void skip_ws() {
    while (!eof()) {
      const int b = peek();
      if (b == ' ' || b == '\n' || b == '\r' || b == '\t') ++pos;
      else break;
    }
  }

  void expect(int want) {
    skip_ws();
    if (eof() || peek() != want)
      fail("JSON_PARSE_ERROR", "expected byte " + S(want) + " at " + S((long long)pos), shard_, "");
    ++pos;
  }

  int64_t parse_uint() {
    skip_ws();
    int64_t v = 0;
    int nd = 0;
    while (!eof()) {
      const int b = peek();
      if (b < '0' || b > '9') break;
      if (v > 900719925474099LL) fail("INVALID_HEADER", "integer overflow", shard_, "");
      v = v * 10 + (b - '0');
      ++nd;
      ++pos;
    }
    if (nd == 0) fail("JSON_PARSE_ERROR", "expected integer at " + S((long long)pos), shard_, "");
    return v;
  }

  std::string parse_string() {
    expect('"');
    std::string out;
    while (true) {
      if (eof()) fail("JSON_PARSE_ERROR", "unterminated string", shard_, "");
      const int b = peek();
      if (b == '"') {
        ++pos;
        break;
      }
      if (b == '\\') {
        ++pos;
        escape(out);
      } else if (b < 32) {
        fail("JSON_PARSE_ERROR", "raw control < 0x20 at " + S((long long)pos), shard_, "");
      } else {
        out += (char)b;
        ++pos;
      }
    }
    return out;
  }

  void expect_literal(const char* w) {
    for (; *w; ++w) {
      if (eof() || peek() != (unsigned char)*w)
        fail("JSON_PARSE_ERROR", "bad literal at " + S((long long)pos), shard_, "");
      ++pos;
    }
  }

  void skip_number() {  // '-'? digits, then no fraction / exponent (subset)
    if (peek() == '-') ++pos;
    parse_uint();
    skip_ws();
    if (!eof()) {
      const int c = peek();
      if (c == '.' || c == 'E' || c == 'e')
        fail("JSON_PARSE_ERROR", "pecahan/eksponen di luar subset", shard_, "");
    }
  }

  void skip_value() {
    skip_ws();
    if (eof()) fail("JSON_PARSE_ERROR", "unexpected eof", shard_, "");
    const int b = peek();
    if (b == '"') {
      parse_string();
      return;
    }
    if ((b >= '0' && b <= '9') || b == '-') {
      skip_number();
      return;
    }
    if (b == 't') { expect_literal("true"); return; }
    if (b == 'f') { expect_literal("false"); return; }
    if (b == 'n') { expect_literal("null"); return; }
    if (b != '{' && b != '[') fail("JSON_PARSE_ERROR", "bad value at " + S((long long)pos), shard_, "");
    std::vector<int> stack{b};
    ++pos;
    while (!stack.empty()) {
      if (eof()) fail("JSON_PARSE_ERROR", "unterminated composite", shard_, "");
      const int c = peek();
      if (c == '"') {
        parse_string();
      } else if (c == '{' || c == '[') {
        stack.push_back(c);
        ++pos;
      } else if (c == '}' || c == ']') {
        const int want = stack.back() == '[' ? ']' : '}';
        if (c != want) fail("JSON_PARSE_ERROR", "tutup silang at " + S((long long)pos), shard_, "");
        stack.pop_back();
        ++pos;
      } else if (c == ',' || c == ':') {
        ++pos;
      } else if ((c >= '0' && c <= '9') || c == '-') {
        skip_number();
      } else if (c == ' ' || c == '\n' || c == '\r' || c == '\t') {
        ++pos;
      } else {
        fail("JSON_PARSE_ERROR", "byte liar at " + S((long long)pos), shard_, "");
      }
    }
  }

  std::vector<int64_t> parse_int_array() {
    std::vector<int64_t> out;
    expect('[');
    skip_ws();
    if (!eof() && peek() == ']') {
      ++pos;
      return out;
    }
    while (true) {
      out.push_back(parse_uint());
      skip_ws();
      if (eof()) fail("JSON_PARSE_ERROR", "unterminated array", shard_, "");
      const int b = peek();
      ++pos;
      if (b == ']') break;
      if (b != ',') fail("JSON_PARSE_ERROR", "expected , or ]", shard_, "");
    }
    return out;
  }

 private:
  // parse_json_escape / parse_hex4_at / append_utf8_cp (src/format/utf8.mojo)
  int hex4() {
    int v = 0;
    for (int i = 0; i < 4; ++i) {
      if (eof()) fail("JSON_PARSE_ERROR", "bad \\u escape", shard_, "");
      const int b = buf_[pos++];
      int d = -1;
      if (b >= '0' && b <= '9') d = b - '0';
      else if (b >= 'A' && b <= 'F') d = b - 55;
      else if (b >= 'a' && b <= 'f') d = b - 87;
      if (d < 0) fail("JSON_PARSE_ERROR", "bad \\u escape", shard_, "");
      v = v * 16 + d;
    }
    return v;
  }
  void escape(std::string& out) {
    if (eof()) fail("JSON_PARSE_ERROR", "bad escape", shard_, "");
    const int e = buf_[pos++];
    switch (e) {
      case '"': out += '"'; return;
      case '\\': out += '\\'; return;
      case '/': out += '/'; return;
      case 'b': out += '\b'; return;
      case 'f': out += '\f'; return;
      case 'n': out += '\n'; return;
      case 'r': out += '\r'; return;
      case 't': out += '\t'; return;
      case 'u': break;
      default: fail("JSON_PARSE_ERROR", "bad escape", shard_, "");
    }
    int cp = hex4();
    if (cp >= 0xD800 && cp <= 0xDBFF) {
      if (pos + 1 >= buf_.size() || buf_[pos] != '\\' || buf_[pos + 1] != 'u')
        fail("JSON_PARSE_ERROR", "lone high surrogate", shard_, "");
      pos += 2;
      const int lo = hex4();
      if (lo < 0xDC00 || lo > 0xDFFF) fail("JSON_PARSE_ERROR", "bad low surrogate", shard_, "");
      cp = 0x10000 + (cp - 0xD800) * 1024 + (lo - 0xDC00);
    } else if (cp >= 0xDC00 && cp <= 0xDFFF) {
      fail("JSON_PARSE_ERROR", "lone low surrogate", shard_, "");
    }
    if (cp < 0x80) {
      out += (char)cp;
    } else if (cp < 0x800) {
      out += (char)(0xC0 + cp / 64);
      out += (char)(0x80 + cp % 64);
    } else if (cp < 0x10000) {
      out += (char)(0xE0 + cp / 4096);
      out += (char)(0x80 + (cp / 64) % 64);
      out += (char)(0x80 + cp % 64);
    } else {
      out += (char)(0xF0 + cp / 262144);
      out += (char)(0x80 + (cp / 4096) % 64);
      out += (char)(0x80 + (cp / 64) % 64);
      out += (char)(0x80 + cp % 64);
    }
  }
  const std::vector<uint8_t>& buf_;
  std::string shard_;
};

struct File {
  FILE* f = nullptr;
  ~File() {
    if (f) fclose(f);
  }
};

bool read_at(FILE* f, int64_t off, void* dst, int64_t n) {
  if (n == 0) return true;
  if (fseeko(f, (off_t)off, SEEK_SET) != 0) return false;
  return fread(dst, 1, (size_t)n, f) == (size_t)n;
}

bool allowed_group(int64_t g) { return g == 32 || g == 64 || g == 128 || g == 256; }

// Python-style remainder (the reference's Int %).
int64_t pymod(int64_t a, int64_t b) {
  const int64_t r = a % b;
  return (r != 0 && ((r < 0) != (b < 0))) ? r + b : r;
}

// ---- quant model ------------------------------------------------------------
constexpr int kQuantHeader = 256;

// BlockHeader.from_bytes (quant_reader.mojo:97-167)
void parse_quant_header(const std::vector<uint8_t>& raw, QuantFile* q) {
  Scanner sc(raw, "quant_header");
  sc.expect('{');
  int64_t version = 1, group = 128, num = 0, total = 0;
  std::string model, format, scale_dtype = "FP16";
  while (true) {
    sc.skip_ws();
    if (sc.peek() == '}') {
      ++sc.pos;
      break;
    }
    const std::string key = sc.parse_string();
    sc.expect(':');
    if (key == "version") {
      version = sc.parse_uint();
    } else if (key == "model") {
      model = sc.parse_string();
    } else if (key == "quantization") {
      sc.expect('{');
      while (true) {
        sc.skip_ws();
        if (sc.peek() == '}') {
          ++sc.pos;
          break;
        }
        const std::string qk = sc.parse_string();
        sc.expect(':');
        if (qk == "format") format = sc.parse_string();
        else if (qk == "group_size") group = sc.parse_uint();
        else if (qk == "scale_dtype") scale_dtype = sc.parse_string();
        else sc.skip_value();
        sc.skip_ws();
        if (sc.peek() == ',') ++sc.pos;
      }
    } else if (key == "num_tensors") {
      num = sc.parse_uint();
    } else if (key == "total_bytes") {
      total = sc.parse_uint();
    } else {
      sc.skip_value();
    }
    sc.skip_ws();
    if (sc.peek() == ',') ++sc.pos;
  }
  q->version = (int)version;
  q->model = model;
  q->format = format;
  q->group_size = (int)group;
  q->scale_dtype = scale_dtype;
  q->num_tensors = num;
  q->total_bytes = total;
}

// validate_block_header (quant_reader.mojo:345-385); throws the message
void validate_quant_header(const QuantFile& h, int64_t file_size) {
  if (h.version != 1)
    throw ParseFail{"Invalid quant header version: expected 1, got " + S(h.version)};
  if (h.group_size <= 0)
    throw ParseFail{"Group size must be positive, got " + S(h.group_size)};
  if (!allowed_group(h.group_size))
    throw ParseFail{"Group size must be one of {32, 64, 128, 256}, got " + S(h.group_size)};
  if (h.format != "4-bit per-group")
    throw ParseFail{"Unsupported quantization format: " + h.format};
  if (h.scale_dtype != "FP16") throw ParseFail{"Unsupported scale dtype: " + h.scale_dtype};
  if (h.num_tensors <= 0)
    throw ParseFail{"Header num_tensors must be positive, got " + S(h.num_tensors)};
  if (h.num_tensors > 100000)
    throw ParseFail{"Header num_tensors exceeds configured max: " + S(h.num_tensors) +
                    " > 100000"};
  if (file_size > 0 && h.total_bytes != file_size)
    throw ParseFail{"File size mismatch: header total_bytes=" + S(h.total_bytes) +
                    ", physical size=" + S(file_size)};
}

// BlockTensorMeta.from_json_bytes + its constructor (quant_reader.mojo:181-210,
// 268-335)
FileTensor parse_quant_meta(const std::vector<uint8_t>& raw) {
  Scanner sc(raw, "tensor_metadata");
  sc.expect('{');
  FileTensor m;
  m.dtype = "BF16";
  m.quantized_dtype = "4-bit";
  int64_t group = 128, num_groups = 0, soff = 0, doff = 0;
  while (true) {
    sc.skip_ws();
    if (sc.peek() == '}') {
      ++sc.pos;
      break;
    }
    const std::string key = sc.parse_string();
    sc.expect(':');
    if (key == "name") {
      m.name = sc.parse_string();
    } else if (key == "shape") {
      sc.expect('[');
      while (true) {
        sc.skip_ws();
        if (sc.peek() == ']') {
          ++sc.pos;
          break;
        }
        m.shape.push_back(sc.parse_uint());
        sc.skip_ws();
        if (sc.peek() == ',') ++sc.pos;
      }
    } else if (key == "dtype") {
      m.dtype = sc.parse_string();
    } else if (key == "quantized_dtype") {
      m.quantized_dtype = sc.parse_string();
    } else if (key == "group_size") {
      group = sc.parse_uint();
    } else if (key == "num_groups") {
      num_groups = sc.parse_uint();
    } else if (key == "scale_offset") {
      soff = sc.parse_uint();
    } else if (key == "data_offset") {
      doff = sc.parse_uint();
    } else {
      sc.skip_value();
    }
    sc.skip_ws();
    if (sc.peek() == ',') ++sc.pos;
  }
  if (!allowed_group(group))
    throw ParseFail{"BlockTensorMeta: group_size not in {32, 64, 128, 256}"};
  uint64_t n = 1;  // the reference's Int product (wraps)
  for (int64_t d : m.shape) n *= (uint64_t)d;
  if (pymod((int64_t)n, group) != 0)
    throw ParseFail{"BlockTensorMeta: N % G != 0 (tail group not supported)"};
  m.group_size = (int)group;
  m.num_groups = num_groups;
  m.scales_offset = soff;  // relative until the record is placed
  m.data_offset = doff;
  return m;
}

// validate_block_tensor_meta (quant_reader.mojo:388-433)
int64_t validate_quant_meta(const FileTensor& m) {
  if (m.name.empty()) throw ParseFail{"Tensor name cannot be empty"};
  if (m.name.size() > 512)
    throw ParseFail{"Tensor name length exceeds configured max: " + S((long long)m.name.size()) +
                    " > 512"};
  if (!allowed_group(m.group_size))
    throw ParseFail{"Group size must be one of {32, 64, 128, 256}, got " + S(m.group_size)};
  if (m.shape.empty()) throw ParseFail{"Tensor shape cannot be empty"};
  if (m.shape.size() > 8)
    throw ParseFail{"Tensor ndim exceeds configured max: " + S((long long)m.shape.size()) +
                    " > 8"};
  int64_t n = 1;
  for (int64_t d : m.shape) {
    if (d <= 0) throw ParseFail{"Dimension must be positive, got " + S(d)};
    if (n > 0x7FFFFFFFFFFFFFFFLL / d)
      throw ParseFail{"safe_multiply_int: integer multiplication overflow"};
    n *= d;
  }
  if (n % m.group_size != 0)
    throw ParseFail{"Tensor num_elements must be divisible by group_size: " + S(n) + " % " +
                    S(m.group_size) + " != 0"};
  const int64_t expected = n / m.group_size;
  if (m.num_groups != expected)
    throw ParseFail{"num_groups mismatch: meta=" + S(m.num_groups) + ", expected=" + S(expected)};
  return n;
}

// ---- safetensors -------------------------------------------------------------
constexpr int64_t kHeaderMax = 100000000;
constexpr int64_t kTensorMax = 100000;

int64_t dtype_size(const std::string& d) {  // types.mojo:169-178
  if (d == "BF16" || d == "F16") return 2;
  if (d == "F32") return 4;
  if (d == "F64") return 8;
  return -1;
}

}  // namespace

std::string error_json(const std::string& type, const std::string& detail,
                       const std::string& shard, const std::string& tensor) {
  return "{\"error_type\":\"" + json_escape(type) + "\",\"detail\":\"" + json_escape(detail) +
         "\",\"shard\":\"" + json_escape(shard) + "\",\"tensor_name\":\"" + json_escape(tensor) +
         "\"}";
}

int QuantFile::find(const std::string& name) const {
  for (int i = (int)tensors.size() - 1; i >= 0; --i)
    if (tensors[i].name == name) return i;
  return -1;
}

int SafetensorsFile::find(const std::string& name) const {
  for (int i = 0; i < (int)tensors.size(); ++i)
    if (tensors[i].name == name) return i;
  return -1;
}

// scan_quant_file (quant_reader.mojo:487-662)
bool scan_quant_file(const std::string& path, QuantFile* out, std::string* err) {
  File fh;
  fh.f = fopen(path.c_str(), "rb");
  if (!fh.f) {
    *err = "scan_quant_file: cannot open " + path;
    return false;
  }
  if (fseeko(fh.f, 0, SEEK_END) != 0) {
    *err = "scan_quant_file: cannot open " + path;
    return false;
  }
  const int64_t file_size = (int64_t)ftello(fh.f);
  if (file_size < kQuantHeader) {
    *err = "scan_quant_file: file truncated, size " + S(file_size) + " < header size " +
           S(kQuantHeader);
    return false;
  }
  QuantFile q;
  q.path = path;
  std::vector<uint8_t> hdr(kQuantHeader);
  if (!read_at(fh.f, 0, hdr.data(), kQuantHeader)) {
    *err = "scan_quant_file: file truncated, size " + S(file_size) + " < header size 256";
    return false;
  }
  try {
    parse_quant_header(hdr, &q);
  } catch (const ParseFail& e) {
    *err = "scan_quant_file: failed parsing quant header: " + e.msg;
    return false;
  }
  try {
    validate_quant_header(q, file_size);
  } catch (const ParseFail& e) {
    *err = "scan_quant_file: header validation failed (SEC-4): " + e.msg;
    return false;
  }
  int64_t cur = kQuantHeader;
  for (int64_t t = 0; t < q.num_tensors; ++t) {
    if (cur + 4 > file_size) {
      *err = "scan_quant_file: framing truncated before meta_len at tensor " + S(t);
      return false;
    }
    uint8_t lb[4];
    if (!read_at(fh.f, cur, lb, 4)) {
      *err = "scan_quant_file: framing truncated before meta_len at tensor " + S(t);
      return false;
    }
    const int64_t meta_len = (int64_t)lb[0] | ((int64_t)lb[1] << 8) | ((int64_t)lb[2] << 16) |
                             ((int64_t)lb[3] << 24);
    if (meta_len <= 0 || cur + 4 + meta_len > file_size) {
      *err = "scan_quant_file: invalid meta_len (" + S(meta_len) + ") at offset " + S(cur);
      return false;
    }
    std::vector<uint8_t> js((size_t)meta_len);
    if (!read_at(fh.f, cur + 4, js.data(), meta_len)) {
      *err = "scan_quant_file: invalid meta_len (" + S(meta_len) + ") at offset " + S(cur);
      return false;
    }
    FileTensor m;
    try {
      m = parse_quant_meta(js);
    } catch (const ParseFail& e) {
      *err = "scan_quant_file: failed parsing tensor metadata JSON at tensor " + S(t) + ": " +
             e.msg;
      return false;
    }
    int64_t n = 0;
    try {
      n = validate_quant_meta(m);
    } catch (const ParseFail& e) {
      *err = "scan_quant_file: tensor metadata failed SEC-4 validation: " + e.msg;
      return false;
    }
    const int64_t s_bytes = m.num_groups * 2, w_bytes = (n + 1) / 2;
    const int64_t rec = 4 + meta_len + s_bytes + w_bytes;
    if (cur + rec > file_size) {
      *err = "scan_quant_file: tensor payload truncated: " + m.name + " (offset " +
             S(cur + rec) + " > " + S(file_size) + ")";
      return false;
    }
    const int64_t payload = cur + 4 + meta_len;
    m.scales_offset = payload + m.scales_offset;
    m.data_offset = payload + m.data_offset;
    m.scales_bytes = s_bytes;
    m.data_bytes = w_bytes;
    q.tensors.push_back(std::move(m));
    cur += rec;
  }
  if (cur != file_size) {
    *err = "scan_quant_file: trailing data or size mismatch (read " + S(cur) +
           " != file_size " + S(file_size) + ")";
    return false;
  }
  *out = std::move(q);
  return true;
}

// pread_tensor_quant (quant_reader.mojo:665-692).  The meta's scale and data
// offsets are not validated by the scan, so reads past the file end fail
// here instead of returning short buffers.
bool read_quant_tensor(const QuantFile& f, int idx, uint16_t* scales, uint8_t* packed,
                       std::string* err) {
  if (idx < 0 || idx >= (int)f.tensors.size()) {
    *err = "pread_tensor_quant: no tensor " + S(idx);
    return false;
  }
  const FileTensor& t = f.tensors[idx];
  File fh;
  fh.f = fopen(f.path.c_str(), "rb");
  if (!fh.f) {
    *err = "pread_tensor_quant: cannot open " + f.path;
    return false;
  }
  std::vector<uint8_t> sb((size_t)t.scales_bytes);
  if (!read_at(fh.f, t.scales_offset, sb.data(), t.scales_bytes) ||
      !read_at(fh.f, t.data_offset, packed, t.data_bytes)) {
    *err = "pread_tensor_quant: short read of " + t.name;
    return false;
  }
  for (int64_t g = 0; g < t.num_groups; ++g)
    scales[g] = (uint16_t)(sb[2 * g] | (sb[2 * g + 1] << 8));
  return true;
}

// read_header (reader.mojo:21-297)
bool read_safetensors_header(const std::string& path, SafetensorsFile* out, std::string* err) {
  try {
    File fh;
    fh.f = fopen(path.c_str(), "rb");
    if (!fh.f) fail("FILE_NOT_FOUND", "tidak bisa open: " + path, path, "");
    fseeko(fh.f, 0, SEEK_END);
    const int64_t filesize = (int64_t)ftello(fh.f);
    uint8_t pre[8];
    if (filesize < 8 || !read_at(fh.f, 0, pre, 8)) fail("INVALID_HEADER", "file < 8 byte", path, "");
    uint64_t hl = 0;
    for (int i = 7; i >= 0; --i) hl = (hl << 8) | pre[i];
    if (hl > (uint64_t)kHeaderMax)
      fail("INVALID_HEADER", "header_len melebihi 100 MB: " + std::to_string(hl), path, "");
    const int64_t header_len = (int64_t)hl, data_base = 8 + header_len;
    if (data_base > filesize) fail("INVALID_HEADER", "header melebihi filesize", path, "");
    std::vector<uint8_t> hb((size_t)header_len);
    if (!read_at(fh.f, 8, hb.data(), header_len)) fail("INVALID_HEADER", "header terpotong", path, "");
    Scanner sc(hb, path);
    sc.skip_ws();
    sc.expect('{');
    SafetensorsFile st;
    st.path = path;
    st.filesize = filesize;
    st.data_base = data_base;
    st.header_len = header_len;
    while (true) {
      sc.skip_ws();
      if (sc.eof()) fail("JSON_PARSE_ERROR", "objek tak berakhir", path, "");
      if (sc.peek() == '}') {
        ++sc.pos;
        break;
      }
      const std::string key = sc.parse_string();
      sc.expect(':');
      if (key == "__metadata__") {
        sc.skip_value();
      } else {
        for (const FileTensor& t : st.tensors)
          if (t.name == key) fail("DUPLICATE_JSON_KEY", "kunci ganda: " + key, path, key);
        sc.skip_ws();
        sc.expect('{');
        FileTensor m;
        m.name = key;
        bool has_dtype = false, has_shape = false, has_off = false;
        int64_t begin = -1, end = -1;
        while (true) {
          sc.skip_ws();
          if (sc.eof()) fail("JSON_PARSE_ERROR", "objek tensor putus", path, key);
          if (sc.peek() == '}') {
            ++sc.pos;
            break;
          }
          const std::string field = sc.parse_string();
          sc.expect(':');
          if (field == "dtype") {
            m.dtype = sc.parse_string();
            has_dtype = true;
          } else if (field == "shape") {
            m.shape = sc.parse_int_array();
            has_shape = true;
          } else if (field == "data_offsets") {
            sc.skip_ws();
            sc.expect('[');
            begin = sc.parse_uint();
            sc.skip_ws();
            sc.expect(',');
            const int64_t e2 = sc.parse_uint();
            sc.skip_ws();
            sc.expect(']');
            end = e2;
            has_off = true;
          } else {
            sc.skip_value();
          }
          sc.skip_ws();
          if (sc.eof()) fail("JSON_PARSE_ERROR", "objek tensor putus", path, key);
          const int c = sc.peek();
          ++sc.pos;
          if (c == '}') break;
          if (c != ',') fail("JSON_PARSE_ERROR", "harap , atau }", path, key);
        }
        if (!has_dtype || !has_shape || !has_off) fail("INVALID_HEADER", "field kurang", path, key);
        const int64_t sz = dtype_size(m.dtype);
        if (sz < 0) fail("UNKNOWN_DTYPE", "dtype asing: " + m.dtype, path, key);
        if (begin < 0 || end < begin)
          fail("OFFSET_OVERFLOW", "BEGIN/END invalid: " + S(begin) + ".." + S(end), path, key);
        if (end > filesize - data_base)
          fail("OFFSET_OVERFLOW",
               "akhir buffer " + S(end) + " + data_base " + S(data_base) + " = file " +
                   S(end + data_base) + " > filesize " + S(filesize),
               path, key);
        int64_t numel = 1;  // _numel_or_fail (types.mojo:199-218)
        for (int64_t d : m.shape) {
          if (d < 0) fail("INVALID_HEADER", "dimensi negatif", path, key);
          if (d > 0 && numel > 4611686018427387903LL / d)
            fail("INVALID_HEADER", "numel overflow", path, key);
          numel *= d;
        }
        if (end - begin != numel * sz)
          fail("LAYOUT_MISMATCH",
               "len " + S(end - begin) + " != numel*size " + S(numel * sz), path, key);
        m.data_offset = begin;  // relative to data_base until the checks pass
        m.data_bytes = end - begin;
        st.tensors.push_back(std::move(m));
      }
      sc.skip_ws();
      if (sc.eof()) fail("JSON_PARSE_ERROR", "objek putus", path, "");
      const int sep = sc.peek();
      ++sc.pos;
      if (sep == '}') break;
      if (sep != ',') fail("JSON_PARSE_ERROR", "harap , atau }", path, "");
    }
    if ((int64_t)st.tensors.size() > kTensorMax)
      fail("INVALID_HEADER", "tensor > 100000", path, "");
    // F15b: sorted by begin, the buffers tile the payload.  The reference's
    // exchange sort decides the order among equal begins; it is kept for
    // headers of up to 20000 tensors (real shards hold far fewer).
    std::vector<int> order(st.tensors.size());
    for (size_t i = 0; i < order.size(); ++i) order[i] = (int)i;
    if (order.size() <= 20000) {
      for (size_t i = 0; i < order.size(); ++i)
        for (size_t j = i + 1; j < order.size(); ++j)
          if (st.tensors[order[j]].data_offset < st.tensors[order[i]].data_offset)
            std::swap(order[i], order[j]);
    } else {
      std::stable_sort(order.begin(), order.end(), [&](int a, int b) {
        return st.tensors[a].data_offset < st.tensors[b].data_offset;
      });
    }
    int64_t prev = 0;
    for (int k : order) {
      const FileTensor& m = st.tensors[k];
      if (m.data_offset != prev)
        fail("OFFSET_OVERFLOW",
             "lubang/overlap di " + S(m.data_offset) + " (harap " + S(prev) + ")", path, m.name);
      prev = m.data_offset + m.data_bytes;
    }
    if (prev != filesize - data_base)
      fail("OFFSET_OVERFLOW",
           "buffer tak penuh: akhir " + S(prev) + " != " + S(filesize - data_base), path, "");
    for (FileTensor& m : st.tensors) m.data_offset += data_base;
    *out = std::move(st);
    return true;
  } catch (const ParseFail& e) {
    *err = e.msg;
    return false;
  }
}

bool read_safetensors_tensor(const SafetensorsFile& f, int idx, void* out, int64_t count,
                             std::string* err) {
  if (idx < 0 || idx >= (int)f.tensors.size()) {
    *err = error_json("TENSOR_NOT_FOUND", "no tensor " + S(idx), f.path, "");
    return false;
  }
  const FileTensor& t = f.tensors[idx];
  if (count != t.data_bytes) {
    *err = error_json("LAYOUT_MISMATCH",
                      "len " + S(t.data_bytes) + " != requested " + S(count), f.path, t.name);
    return false;
  }
  File fh;
  fh.f = fopen(f.path.c_str(), "rb");
  if (!fh.f || !read_at(fh.f, t.data_offset, out, count)) {
    *err = error_json("FILE_NOT_FOUND", "tidak bisa open: " + f.path, f.path, t.name);
    return false;
  }
  return true;
}

}  // namespace dm
