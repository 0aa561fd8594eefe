// qnn_files.cpp -- safetensors and GGUF tensor tables, mapped read-only.
//
// Restates the reference's checkpoint readers:
//  * TSafeTensorFile.Open (src/io/QuickNN.SafeTensors.pas:522-690): an 8-byte
//    header length, a UTF-8 JSON header of tensor descriptors, then one data
//    buffer that the descriptors must tile exactly;
//  * TGGUFHeader.Read (src/io/QuickNN.GGUF.pas:206-337) and OpenGGUF
//    (SafeTensors.pas:480-520): GGUF v2/v3 metadata and tensor table;
//  * LoadSafeTensorShards (SafeTensors.pas:777-837) and GetTensor /
//    GetLinearWeight (:874-912).
// The limits, checks and their order follow those lines, so a file the
// reference rejects is rejected here with QNN_E_FORMAT.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <map>
#include <sstream>

#include "qnn_formats.h"

namespace qnn {
namespace fmt {

Mapping::~Mapping() {
  if (addr && size) munmap(addr, size);
}

uint64_t new_identity() {
  static std::atomic<uint64_t> next{1};
  return (uint64_t(1) << 63) | next.fetch_add(1);
}

bool file_exists(const std::string &path) {
  struct stat st;
  return stat(path.c_str(), &st) == 0 && S_ISREG(st.st_mode);
}

std::string join_path(const std::string &dir, const std::string &name) {
  if (dir.empty()) return name;
  if (!name.empty() && name[0] == '/') return name;
  return dir.back() == '/' ? dir + name : dir + "/" + name;
}

std::string full_path(const std::string &path) {
  std::string p = path;
  if (p.empty() || p[0] != '/') {
    char cwd[4096];
    if (!getcwd(cwd, sizeof cwd)) fail(QNN_E_IO, "cannot read the working directory");
    p = join_path(cwd, p);
  }
  std::vector<std::string> parts;
  std::stringstream ss(p);
  std::string seg;
  while (std::getline(ss, seg, '/')) {
    if (seg.empty() || seg == ".") continue;
    if (seg == "..") {
      if (!parts.empty()) parts.pop_back();
      continue;
    }
    parts.push_back(seg);
  }
  std::string out;
  for (const auto &s : parts) out += "/" + s;
  return out.empty() ? "/" : out;
}

std::string read_text(const std::string &path) {
  std::ifstream f(path, std::ios::binary);
  if (!f) fail(QNN_E_IO, "cannot open " + path);
  std::string s((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
  if (s.size() >= 3 && (unsigned char)s[0] == 0xEF && (unsigned char)s[1] == 0xBB && (unsigned char)s[2] == 0xBF)
    s.erase(0, 3);
  return s;
}

namespace {

constexpr uint32_t kGgufMagic = 0x46554747u;  // "GGUF"

// DTYPE_NAMES and TSafeTensorTypeHelper.Bits / ToDataType
// (SafeTensors.pas:79-132, :298-333), indexed by TSafeTensorType ordinal.
struct StType {
  const char *name;
  int bits;
  int dt;
};
const StType kStTypes[] = {
    {"BOOL", 8, QNN_DT_BOOLEAN},   {"F4", 4, QNN_DT_F4E2M1},     {"F6_E2M3", 6, QNN_DT_UNDEF},
    {"F6_E3M2", 6, QNN_DT_UNDEF},  {"U8", 8, QNN_DT_U8},         {"I8", 8, QNN_DT_S8},
    {"F8_E5M2", 8, QNN_DT_F8E5M2}, {"F8_E4M3", 8, QNN_DT_F8E4M3}, {"F8_E8M0", 8, QNN_DT_UNDEF},
    {"I16", 16, QNN_DT_S16},       {"U16", 16, QNN_DT_U16},      {"F16", 16, QNN_DT_F16},
    {"BF16", 16, QNN_DT_BF16},     {"I32", 32, QNN_DT_S32},      {"U32", 32, QNN_DT_UNDEF},
    {"F32", 32, QNN_DT_F32},       {"C64", 64, QNN_DT_UNDEF},    {"F64", 64, QNN_DT_F64},
    {"I64", 64, QNN_DT_UNDEF},     {"U64", 64, QNN_DT_UNDEF},    {"I4", 4, QNN_DT_S4},
};
constexpr int kStTypeCount = int(sizeof(kStTypes) / sizeof(kStTypes[0]));

int st_from_string(const std::string &s) {
  for (int i = 0; i < kStTypeCount; ++i)
    if (s == kStTypes[i].name) return i;
  return QNN_ST_UNKNOWN;
}
int st_bits(int t) { return t >= 0 && t < kStTypeCount ? kStTypes[t].bits : 0; }
int st_datatype(int t) { return t >= 0 && t < kStTypeCount ? kStTypes[t].dt : QNN_DT_UNDEF; }

// GGUFEncoding / GGUFBlockElements / GGUFBlockBytes
// (src/io/QuickNN.GGUF.Quantization.pas:44-99).
int gguf_encoding(uint32_t storage) {
  switch (storage) {
    case 16: return QNN_WE_IQ2_XXS;
    case 18: return QNN_WE_IQ3_XXS;
    case 22: return QNN_WE_IQ2_S;
    case 42: return QNN_WE_Q2_0;
    case 8: return QNN_WE_Q8_0;
    case 10: return QNN_WE_Q2_K;
    case 12: return QNN_WE_Q4_K;
    case 14: return QNN_WE_Q6_K;
    case 11: return QNN_WE_Q3_K;
    case 13: return QNN_WE_Q5_K;
    case 20: return QNN_WE_IQ4_NL;
    case 21: return QNN_WE_IQ3_S;
    case 23: return QNN_WE_IQ4_XS;
    default: return QNN_WE_NATIVE;
  }
}
int block_elements(int enc) {
  switch (enc) {
    case QNN_WE_Q2_0: return 64;
    case QNN_WE_Q8_0: case QNN_WE_IQ4_NL: return 32;
    default: return 256;
  }
}
int block_bytes(int enc) {
  switch (enc) {
    case QNN_WE_IQ3_XXS: return 98;
    case QNN_WE_IQ2_XXS: return 66;
    case QNN_WE_IQ2_S: return 82;
    case QNN_WE_Q2_0: return 18;
    case QNN_WE_Q8_0: return 34;
    case QNN_WE_Q2_K: return 84;
    case QNN_WE_Q4_K: return 144;
    case QNN_WE_Q6_K: return 210;
    case QNN_WE_Q3_K: case QNN_WE_IQ3_S: return 110;
    case QNN_WE_Q5_K: return 176;
    case QNN_WE_IQ4_NL: return 18;
    case QNN_WE_IQ4_XS: return 136;
    default: return 0;
  }
}

std::string dec_u32(uint32_t v) {
  char b[16];
  std::snprintf(b, sizeof b, "%u", v);
  return b;
}

// An open file descriptor, closed on scope exit.
struct Fd {
  int fd = -1;
  ~Fd() {
    if (fd >= 0) close(fd);
  }
};

std::shared_ptr<Mapping> map_file(int fd, int64_t size, const std::string &what) {
  auto m = std::make_shared<Mapping>();
  void *p = mmap(nullptr, size_t(size), PROT_READ, MAP_PRIVATE, fd, 0);
  if (p == MAP_FAILED) fail(QNN_E_FORMAT, "Unable to map " + what);
  m->addr = p;
  m->size = size_t(size);
  return m;
}

}  // namespace

// ---------------------------------------------------------------------------
// GGUF header (src/io/QuickNN.GGUF.pas:44-337)
// ---------------------------------------------------------------------------
struct GgufTensor {
  std::string name;
  std::vector<int64_t> shape;
  uint32_t storage = 0;
  int encoding = QNN_WE_NATIVE;
  int64_t offset = 0, byte_size = 0;
};

struct GgufHeader {
  uint32_t version = 0, alignment = 32;
  std::string architecture;
  int64_t data_offset = 0;
  int32_t vocabulary_size = 0;
  std::vector<GgufTensor> tensors;
  std::string metadata_json;
};

namespace {

constexpr int64_t kMaxHeaderBytes = 100000000;
constexpr uint64_t kMaxItems = 1000000;
constexpr uint64_t kMaxStringBytes = 16ull * 1024 * 1024;

class GgufReader {
 public:
  GgufReader(const uint8_t *base, int64_t size) : base_(base), size_(size) {}

  GgufHeader read(bool with_metadata, bool include_vocabulary) {
    GgufHeader h;
    if (u32() != kGgufMagic) err("Invalid GGUF magic (only little-endian GGUF is supported)");
    h.version = u32();
    if (h.version != 2 && h.version != 3) err("Unsupported GGUF version " + dec_u32(h.version));
    const uint64_t tensor_count = u64(), metadata_count = u64();
    if (tensor_count > kMaxItems || metadata_count > kMaxItems) err("Too many GGUF tensors or metadata entries");
    h.alignment = 32;
    std::map<std::string, bool> names;
    std::string meta = "{";
    bool first_meta = true;
    auto add_meta = [&](const std::string &key, const std::string &value_json) {
      if (!first_meta) meta += ",";
      first_meta = false;
      meta += json::quote(key) + ":" + value_json;
    };
    for (uint64_t i = 0; i < metadata_count; ++i) {
      const std::string key = read_string();
      if (key.empty() || names.count(key)) err("Empty or duplicate GGUF metadata key");
      names[key] = true;
      const uint32_t kind = u32();
      if (key == "general.architecture") {
        if (kind != 8) err("GGUF architecture must be a string");
        h.architecture = read_string();
        if (with_metadata) add_meta(key, json::quote(h.architecture));
      } else if (key == "general.alignment") {
        if (kind != 4) err("GGUF alignment must be UINT32");
        h.alignment = u32();
        if (h.alignment == 0 || h.alignment > 65536 || (h.alignment & (h.alignment - 1)) != 0)
          err("Invalid GGUF alignment");
      } else if (key == "tokenizer.ggml.tokens" && !include_vocabulary) {
        if (kind != 9 || u32() != 8) err("Invalid GGUF vocabulary");
        const uint64_t count = u64();
        if (count > kMaxItems) err("Oversized GGUF vocabulary");
        h.vocabulary_size = int32_t(count);
        for (uint64_t j = 0; j < count; ++j) skip_string();
      } else if (key == "tokenizer.ggml.merges" && !include_vocabulary) {
        if (kind != 9 || u32() != 8) err("Invalid GGUF merges");
        const uint64_t count = u64();
        if (count > kMaxItems) err("Oversized GGUF merges");
        for (uint64_t j = 0; j < count; ++j) skip_string();
      } else if (with_metadata && (include_vocabulary || (!starts_with(key, "tokenizer.ggml.merges") &&
                                                          !starts_with(key, "tokenizer.ggml.token_type") &&
                                                          !starts_with(key, "tokenizer.ggml.scores")))) {
        int64_t items = -1;
        const std::string v = read_value(kind, 0, &items);
        add_meta(key, v);
        if (key == "tokenizer.ggml.tokens" && kind == 9) h.vocabulary_size = int32_t(items);
      } else {
        skip_value(kind, 0);
      }
    }
    meta += "}";
    if (with_metadata) h.metadata_json = meta;

    names.clear();
    h.tensors.resize(size_t(tensor_count));
    for (auto &t : h.tensors) {
      t.name = read_string();
      if (t.name.empty() || names.count(t.name)) err("Empty or duplicate GGUF tensor name");
      names[t.name] = true;
      const uint32_t dims = u32();
      if (dims < 1 || dims > 4) err("Invalid GGUF tensor rank");
      t.shape.assign(dims, 0);
      int64_t elements = 1;
      for (uint32_t j = 0; j < dims; ++j) {
        const uint64_t d = u64();
        if (d == 0 || d > uint64_t(INT64_MAX) || elements > INT64_MAX / int64_t(d))
          err("Invalid or overflowing GGUF tensor shape");
        t.shape[dims - 1 - j] = int64_t(d);
        elements *= int64_t(d);
      }
      t.storage = u32();
      t.encoding = gguf_encoding(t.storage);
      int element_bytes;
      switch (t.storage) {
        case 0: element_bytes = 4; break;
        case 1: case 30: element_bytes = 2; break;
        case 8: case 10: case 11: case 12: case 13: case 14: case 16: case 18: case 20: case 21: case 22: case 23:
        case 42: element_bytes = 0; break;
        default:
          err("GGUF tensor \"" + t.name + "\": storage type " + dec_u32(t.storage) +
              " is not supported; unsupported GGML block encoding");
      }
      if (t.encoding != QNN_WE_NATIVE) {
        const int64_t be = block_elements(t.encoding), bb = block_bytes(t.encoding);
        if (t.shape.back() % be != 0) err("GGUF row is not a complete quantization block: " + t.name);
        if (uint64_t(elements / be) > uint64_t(INT64_MAX) / uint64_t(bb)) err("GGUF compressed byte size overflow");
        t.byte_size = elements / be * bb;
      } else {
        if (elements > INT64_MAX / element_bytes) err("GGUF tensor byte size overflow");
        t.byte_size = elements * element_bytes;
      }
      const uint64_t off = u64();
      if (off > uint64_t(INT64_MAX) || off % h.alignment != 0) err("Invalid GGUF tensor offset");
      t.offset = int64_t(off);
    }
    const int64_t position = pos_;
    h.data_offset = (position + h.alignment - 1) / h.alignment * h.alignment;
    if (h.data_offset > size_) err("Truncated GGUF alignment padding");
    // Padding between tensors is allowed; overlaps and truncated payloads are not.
    std::vector<const GgufTensor *> sorted;
    for (const auto &t : h.tensors) sorted.push_back(&t);
    std::stable_sort(sorted.begin(), sorted.end(),
                     [](const GgufTensor *a, const GgufTensor *b) { return a->offset < b->offset; });
    int64_t end_offset = 0;
    const int64_t payload = size_ - h.data_offset;
    for (const GgufTensor *t : sorted) {
      if (t->offset < end_offset || t->offset > payload || t->byte_size > payload - t->offset)
        err("Overlapping or truncated GGUF tensor: " + t->name);
      end_offset = t->offset + t->byte_size;
    }
    return h;
  }

 private:
  const uint8_t *base_;
  int64_t size_, pos_ = 0;

  [[noreturn]] static void err(const std::string &m) { fail(QNN_E_FORMAT, m); }
  static bool starts_with(const std::string &s, const char *p) { return s.rfind(p, 0) == 0; }

  void require(int64_t n) {
    if (n < 0 || n > size_ - pos_ || n > kMaxHeaderBytes - pos_) err("Truncated or oversized GGUF header");
  }
  void require_u(uint64_t n) {
    if (n > uint64_t(INT64_MAX)) err("Truncated or oversized GGUF header");
    require(int64_t(n));
  }
  uint64_t bytes_le(int n) {
    require(n);
    uint64_t v = 0;
    for (int i = 0; i < n; ++i) v |= uint64_t(base_[pos_ + i]) << (8 * i);
    pos_ += n;
    return v;
  }
  uint32_t u32() { return uint32_t(bytes_le(4)); }
  uint64_t u64() { return bytes_le(8); }
  std::string read_string() {
    const uint64_t n = u64();
    if (n > kMaxStringBytes) err("Oversized GGUF string");
    require_u(n);
    std::string s(reinterpret_cast<const char *>(base_ + pos_), size_t(n));
    pos_ += int64_t(n);
    if (!json::valid_utf8(s.data(), s.size())) err("Invalid UTF-8 in GGUF header");
    return s;
  }
  void skip_string() {
    const uint64_t n = u64();
    if (n > kMaxStringBytes) err("Oversized GGUF string");
    require_u(n);
    pos_ += int64_t(n);
  }
  static int scalar_bytes(uint32_t kind) {
    switch (kind) {
      case 0: case 1: case 7: return 1;
      case 2: case 3: return 2;
      case 4: case 5: case 6: return 4;
      case 10: case 11: case 12: return 8;
      default: return 0;
    }
  }
  static std::string num_text(double v, int digits) {
    if (!std::isfinite(v)) return "null";
    char b[64];
    std::snprintf(b, sizeof b, "%.*g", digits, v);
    return b;
  }
  // ReadValue (GGUF.pas:112-160): the value as JSON text.
  std::string read_value(uint32_t kind, int depth, int64_t *items = nullptr) {
    if (depth > 16) err("Excessive GGUF metadata nesting");
    if (kind == 8) return json::quote(read_string());
    if (kind == 9) {
      const uint32_t et = u32();
      const uint64_t count = u64();
      if (count > kMaxItems || et > 12 || et == 9) err("Invalid GGUF metadata array");
      if (items) *items = int64_t(count);
      std::string o = "[";
      for (uint64_t i = 0; i < count; ++i) {
        if (i) o += ",";
        o += read_value(et, depth + 1);
      }
      return o + "]";
    }
    const int size = scalar_bytes(kind);
    if (!size) err("Unknown GGUF metadata type");
    const uint64_t bits = bytes_le(size);
    char b[32];
    switch (kind) {
      case 1: std::snprintf(b, sizeof b, "%d", int(int8_t(bits))); return b;
      case 3: std::snprintf(b, sizeof b, "%d", int(int16_t(bits))); return b;
      case 5: std::snprintf(b, sizeof b, "%d", int32_t(bits)); return b;
      case 11: std::snprintf(b, sizeof b, "%lld", (long long)int64_t(bits)); return b;
      case 6: {
        float f;
        const uint32_t u = uint32_t(bits);
        std::memcpy(&f, &u, 4);
        return num_text(f, 9);
      }
      case 12: {
        double d;
        std::memcpy(&d, &bits, 8);
        return num_text(d, 17);
      }
      case 7:
        if (bits > 1) err("Invalid GGUF Boolean");
        return bits ? "true" : "false";
      default: std::snprintf(b, sizeof b, "%llu", (unsigned long long)bits); return b;
    }
  }
  // SkipValue (GGUF.pas:162-204).
  void skip_value(uint32_t kind, int depth) {
    if (depth > 16) err("Excessive GGUF metadata nesting");
    int64_t size = 0;
    if (kind == 8) {
      read_string();
      return;
    }
    if (kind == 9) {
      const uint32_t et = u32();
      const uint64_t count = u64();
      if (count > kMaxItems) err("Oversized GGUF metadata array");
      const int item = scalar_bytes(et);
      if (item > 0) {
        require(int64_t(count) * item);
        pos_ += int64_t(count) * item;
        return;
      }
      if (count > 0) {
        for (uint64_t i = 0; i < count; ++i) skip_value(et, depth + 1);
      } else if (et > 12) {
        err("Unknown GGUF array element type");
      }
      return;
    }
    size = scalar_bytes(kind);
    if (!size) err("Unknown GGUF metadata type " + dec_u32(kind));
    require(size);
    pos_ += size;
  }
};

void sort_by_name(File &f) {
  f.by_name.resize(f.tensors.size());
  for (size_t i = 0; i < f.tensors.size(); ++i) f.by_name[i] = int(i);
  std::sort(f.by_name.begin(), f.by_name.end(),
            [&](int a, int b) { return f.tensors[a].name < f.tensors[b].name; });
}

// OpenGGUF (SafeTensors.pas:480-520).
void open_gguf(File &f, int fd) {
  f.map = map_file(fd, f.file_size, f.path);
  GgufReader r(static_cast<const uint8_t *>(f.map->addr), f.file_size);
  GgufHeader h = r.read(false, false);
  f.is_gguf = true;
  f.architecture = h.architecture;
  f.offset = h.data_offset;
  f.header_size = f.offset;
  f.data_size = f.file_size - f.offset;
  f.tensors.resize(h.tensors.size());
  for (size_t i = 0; i < h.tensors.size(); ++i) {
    const GgufTensor &s = h.tensors[i];
    Tensor &t = f.tensors[i];
    t.name = s.name;
    t.shape = s.shape;
    t.identity = new_identity();
    t.encoding = s.encoding;
    t.storage_type = s.storage;
    switch (s.storage) {
      case 0: t.st_dtype = QNN_ST_F32; break;
      case 1: t.st_dtype = QNN_ST_F16; break;
      case 30: t.st_dtype = QNN_ST_BF16; break;
      default: t.st_dtype = QNN_ST_U8; break;
    }
    t.data_offset = f.offset + s.offset;
    t.data_size = s.byte_size;
    t.data = static_cast<const uint8_t *>(f.map->addr) + t.data_offset;
  }
  sort_by_name(f);
}

}  // namespace

const Tensor *File::find(const std::string &name) const {
  auto it = std::lower_bound(by_name.begin(), by_name.end(), name,
                             [&](int i, const std::string &n) { return tensors[i].name < n; });
  if (it != by_name.end() && tensors[*it].name == name) return &tensors[*it];
  return nullptr;
}

const Tensor *FileSet::find(const std::string &name, int *file_index) const {
  for (size_t i = 0; i < files.size(); ++i)
    if (const Tensor *t = files[i]->find(name)) {
      if (file_index) *file_index = int(i);
      return t;
    }
  return nullptr;
}

// TSafeTensorFile.Open (SafeTensors.pas:522-690).
std::unique_ptr<File> open_file(const std::string &path) {
  constexpr uint64_t kMaxHeaderSize = 100000000;
  auto f = std::make_unique<File>();
  f->path = path;
  Fd fd;
  fd.fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd.fd < 0) fail(QNN_E_IO, "Cannot open file \"" + path + "\": " + std::strerror(errno));
  struct stat st;
  if (fstat(fd.fd, &st) != 0 || !S_ISREG(st.st_mode)) fail(QNN_E_IO, "Cannot open file \"" + path + "\"");
  f->file_size = int64_t(st.st_size);
  auto err = [&](const std::string &m) { fail(QNN_E_FORMAT, m); };
  if (f->file_size < 8) err("Invalid file size or insufficient address space: " + path);
  uint64_t header_length = 0;
  if (pread(fd.fd, &header_length, 8, 0) != 8) fail(QNN_E_IO, "Cannot read " + path);
  if (uint32_t(header_length & 0xffffffffu) == kGgufMagic) {
    open_gguf(*f, fd.fd);
    return f;
  }
  if (header_length < 2 || header_length > kMaxHeaderSize || header_length > uint64_t(f->file_size - 8))
    err("Invalid safetensors header length: " + path);
  f->header_size = int64_t(header_length);
  f->header_json.resize(size_t(header_length));
  if (pread(fd.fd, &f->header_json[0], size_t(header_length), 8) != ssize_t(header_length))
    fail(QNN_E_IO, "Cannot read " + path);
  // The header is parsed as UTF-8 text, never through a code page.
  if (!json::valid_utf8(f->header_json.data(), f->header_json.size())) err("Safetensors header is not valid UTF-8");
  json::Parser parser(f->header_json.data(), f->header_json.size());
  if (!parser.parse(f->json) || !f->json.is_object()) err("Safetensors header must be a JSON object: " + path);
  f->offset = 8 + f->header_size;
  f->data_size = f->file_size - f->offset;
  for (const auto &item : f->json.members) {
    if (item.first == "__metadata__") {
      if (!item.second.is_object()) err("Invalid safetensors metadata");
      for (const auto &m : item.second.members)
        if (!m.second.is_string()) err("Safetensors metadata values must be strings");
      continue;
    }
    if (!item.second.is_object()) err("Invalid tensor descriptor: " + item.first);
    const json::Value &d = item.second;
    const json::Value *offsets = d.get("data_offsets"), *dims = d.get("shape"), *dtype = d.get("dtype");
    if (!offsets || !offsets->is_array() || !dims || !dims->is_array()) err("Invalid tensor offsets or shape");
    if (offsets->items.size() != 2 || !dtype || !dtype->is_string())
      err("Missing tensor descriptor fields: " + item.first);
    Tensor t;
    t.identity = new_identity();
    t.name = item.first;
    t.st_dtype = st_from_string(dtype->text);
    const int bits = st_bits(t.st_dtype);
    if (bits == 0) err("Unknown safetensors dtype: " + dtype->text);
    int64_t first, last;
    auto int_of = [&](const json::Value &v, int64_t &o) {
      if (!v.is_number()) err("Expected an integer in safetensors header");
      if (!v.to_int64(o)) err("Invalid integer in safetensors header");
    };
    int_of(offsets->items[0], first);
    int_of(offsets->items[1], last);
    if (first < 0 || last < first || last > f->data_size)
      err("Tensor offsets are outside the data buffer: " + t.name);
    int64_t elements = 1;
    t.shape.resize(dims->items.size());
    for (size_t j = 0; j < dims->items.size(); ++j) {
      int_of(dims->items[j], t.shape[j]);
      if (t.shape[j] < 0) err("Negative tensor dimension: " + t.name);
      if (t.shape[j] != 0 && elements > INT64_MAX / t.shape[j]) err("Tensor shape overflow: " + t.name);
      elements *= t.shape[j];
    }
    if (elements > INT64_MAX / bits) err("Tensor byte size overflow: " + t.name);
    const int64_t total_bits = elements * bits;
    if (total_bits % 8 != 0 || total_bits / 8 != last - first)
      err("Tensor size does not match shape and dtype: " + t.name);
    t.data_offset = f->offset + first;
    t.data_size = last - first;
    f->tensors.push_back(std::move(t));
  }
  // The descriptors must tile the data buffer exactly, in whatever order they are listed.
  std::vector<int> order(f->tensors.size());
  for (size_t i = 0; i < order.size(); ++i) order[i] = int(i);
  std::sort(order.begin(), order.end(), [&](int a, int b) {
    const Tensor &x = f->tensors[a], &y = f->tensors[b];
    return x.data_offset != y.data_offset ? x.data_offset < y.data_offset : x.data_size < y.data_size;
  });
  int64_t expected_end = f->offset;
  for (int i : order) {
    if (f->tensors[i].data_offset != expected_end) err("Overlapping tensors or a gap in the data buffer");
    expected_end += f->tensors[i].data_size;
  }
  if (expected_end != f->file_size) err("Safetensors data buffer is incomplete or has trailing bytes");
  sort_by_name(*f);
  for (size_t i = 1; i < f->by_name.size(); ++i)
    if (f->tensors[f->by_name[i - 1]].name == f->tensors[f->by_name[i]].name) err("Duplicate tensor name");
  f->map = map_file(fd.fd, f->file_size, path);
  for (auto &t : f->tensors) t.data = static_cast<const uint8_t *>(f->map->addr) + t.data_offset;
  return f;
}

// LoadSafeTensorShards (SafeTensors.pas:777-837).
std::unique_ptr<FileSet> open_shards(const std::string &dir, const std::string &index_file,
                                     const std::string &single_file) {
  auto set = std::make_unique<FileSet>();
  const std::string index_path = join_path(dir, index_file);
  if (index_file.empty() || !file_exists(index_path)) {
    set->files.push_back(open_file(join_path(dir, single_file)));
    return set;
  }
  const std::string text = read_text(index_path);
  json::Value index;
  json::Parser parser(text.data(), text.size());
  if (!parser.parse(index) || !index.is_object()) fail(QNN_E_FORMAT, "Invalid safetensors shard index");
  const json::Value *weights = index.get("weight_map");
  if (!weights || !weights->is_object()) fail(QNN_E_FORMAT, "Missing weight_map in safetensors shard index");
  if (weights->members.empty()) fail(QNN_E_FORMAT, "Empty safetensors shard index");
  std::vector<std::string> files;
  for (const auto &m : weights->members) {
    if (!m.second.is_string() || m.second.text.empty()) fail(QNN_E_FORMAT, "Invalid shard filename");
    if (std::find(files.begin(), files.end(), m.second.text) == files.end()) files.push_back(m.second.text);
  }
  for (const auto &name : files) set->files.push_back(open_file(join_path(dir, name)));
  return set;
}

}  // namespace fmt
}  // namespace qnn

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
struct qnn_gguf_header_s : qnn::fmt::GgufHeader {};

using namespace qnn::fmt;

namespace {

void fill_info(const Tensor &t, int file, qnn_tensor_info *o) {
  o->name = t.name.c_str();
  o->data = t.data;
  o->shape = t.shape.data();
  o->identity = t.identity;
  o->data_offset = t.data_offset;
  o->data_size = t.data_size;
  o->ndim = int32_t(t.shape.size());
  o->st_dtype = t.st_dtype;
  o->dtype = st_datatype(t.st_dtype);
  o->encoding = t.encoding;
  o->file = file;
  o->storage_type = t.storage_type;
}

uint16_t half_bits(const uint8_t *p) { return uint16_t(p[0] | (p[1] << 8)); }
float half_to_float(uint16_t h) {
  const uint32_t sign = uint32_t(h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 0x3ffu;
  uint32_t u;
  if (e == 0) {
    const float v = float(m) * 5.9604644775390625e-8f;  // m * 2^-24, exact
    std::memcpy(&u, &v, 4);
    u |= sign;
  } else if (e == 31) {
    u = sign | 0x7f800000u | (m << 13);
  } else {
    u = sign | ((e + 112) << 23) | (m << 13);
  }
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

void set_shape(qnn_weight *w, const std::vector<int64_t> &shape, int64_t count) {
  w->shape0 = shape.empty() ? 1 : shape[0];
  w->shape1 = shape.size() < 2 ? 1 : (shape[0] ? count / shape[0] : 0);
}

}  // namespace

extern "C" {

int qnn_tensor_files_open(const char *path, qnn_tensor_files **out) {
  return guarded([&] {
    if (!path || !out) fail(QNN_E_ARGUMENT, "null argument");
    *out = nullptr;
    auto set = std::make_unique<qnn_tensor_files_s>();
    set->files.push_back(open_file(path));
    *out = set.release();
    return QNN_OK;
  });
}

int qnn_tensor_files_open_shards(const char *dir, const char *index_file, const char *single_file,
                                 qnn_tensor_files **out) {
  return guarded([&] {
    if (!dir || !out) fail(QNN_E_ARGUMENT, "null argument");
    *out = nullptr;
    auto loaded = open_shards(dir, index_file ? index_file : "", single_file ? single_file : "");
    auto set = std::make_unique<qnn_tensor_files_s>();
    set->files = std::move(loaded->files);
    *out = set.release();
    return QNN_OK;
  });
}

int qnn_tensor_files_close(qnn_tensor_files *files) {
  delete files;
  return QNN_OK;
}

int qnn_tensor_files_count(const qnn_tensor_files *files, int *count) {
  if (!files || !count) return QNN_E_ARGUMENT;
  *count = int(files->files.size());
  return QNN_OK;
}

int qnn_tensor_files_file(const qnn_tensor_files *files, int file, qnn_tensor_file_info *o) {
  return guarded([&] {
    if (!files || !o || file < 0 || file >= int(files->files.size())) fail(QNN_E_ARGUMENT, "file index");
    const File &f = *files->files[file];
    o->path = f.path.c_str();
    o->architecture = f.architecture.c_str();
    o->header_json = f.header_json.c_str();
    o->data = f.map ? f.map->addr : nullptr;
    o->file_size = f.file_size;
    o->header_size = f.header_size;
    o->data_size = f.data_size;
    o->offset = f.offset;
    o->is_gguf = f.is_gguf ? 1 : 0;
    o->tensor_count = int32_t(f.tensors.size());
    return QNN_OK;
  });
}

int qnn_tensor_files_tensor(const qnn_tensor_files *files, int file, int index, qnn_tensor_info *o) {
  return guarded([&] {
    if (!files || !o || file < 0 || file >= int(files->files.size())) fail(QNN_E_ARGUMENT, "file index");
    const File &f = *files->files[file];
    if (index < 0 || index >= int(f.tensors.size())) fail(QNN_E_ARGUMENT, "tensor index");
    fill_info(f.tensors[index], file, o);
    return QNN_OK;
  });
}

int qnn_tensor_files_find(const qnn_tensor_files *files, const char *name, qnn_tensor_info *o) {
  return guarded([&] {
    if (!files || !name || !o) fail(QNN_E_ARGUMENT, "null argument");
    int file = -1;
    const Tensor *t = files->find(name, &file);
    if (!t) return QNN_NOT_FOUND;
    fill_info(*t, file, o);
    return QNN_OK;
  });
}

int qnn_tensor_files_linear_weight(qnn_tensor_files *files, const char *name, qnn_weight *o) {
  return guarded([&] {
    if (!files || !name || !o) fail(QNN_E_ARGUMENT, "null argument");
    int fi = -1;
    const Tensor *t = files->find(name, &fi);
    if (!t) fail(QNN_E_FORMAT, std::string("Cannot find linear weight \"") + name + "\"");
    std::memset(o, 0, sizeof *o);
    o->identity = t->identity;
    o->encoding = t->encoding;
    const int64_t count = t->count();
    set_shape(o, t->shape, count);
    o->size = count;
    if (t->encoding != QNN_WE_NATIVE) {
      o->dtype = QNN_DT_U8;
      o->data = t->data;
      return QNN_OK;
    }
    switch (t->st_dtype) {
      case QNN_ST_BF16: o->dtype = QNN_DT_BF16; o->data = t->data; return QNN_OK;
      case QNN_ST_F32: o->dtype = QNN_DT_F32; o->data = t->data; return QNN_OK;
      case QNN_ST_F16: {
        File &f = *files->files[fi];
        const int idx = int(t - f.tensors.data());
        for (const auto &c : f.converted)
          if (c.first == idx) {
            o->dtype = QNN_DT_F32;
            o->data = c.second.get();
            return QNN_OK;
          }
        std::unique_ptr<float[]> buf(new float[size_t(std::max<int64_t>(count, 1))]);
        for (int64_t i = 0; i < count; ++i) buf[i] = half_to_float(half_bits(t->data + 2 * i));
        o->dtype = QNN_DT_F32;
        o->data = buf.get();
        f.converted.emplace_back(idx, std::move(buf));
        return QNN_OK;
      }
      default:
        fail(QNN_E_FORMAT, "Unsupported conversion to F32: " + t->name);
    }
  });
}

int qnn_gguf_read_file(const char *path, int with_metadata, int include_vocabulary, qnn_gguf_header **out) {
  return guarded([&] {
    if (!path || !out) fail(QNN_E_ARGUMENT, "null argument");
    *out = nullptr;
    Fd fd;
    fd.fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd.fd < 0) fail(QNN_E_IO, std::string("Cannot open file \"") + path + "\": " + std::strerror(errno));
    struct stat st;
    if (fstat(fd.fd, &st) != 0 || !S_ISREG(st.st_mode)) fail(QNN_E_IO, std::string("Cannot open file \"") + path + "\"");
    auto h = std::make_unique<qnn_gguf_header_s>();
    if (st.st_size > 0) {
      auto m = map_file(fd.fd, int64_t(st.st_size), path);
      GgufReader r(static_cast<const uint8_t *>(m->addr), int64_t(st.st_size));
      static_cast<GgufHeader &>(*h) = r.read(with_metadata != 0, include_vocabulary != 0);
    } else {
      fail(QNN_E_FORMAT, "Truncated or oversized GGUF header");
    }
    *out = h.release();
    return QNN_OK;
  });
}

int qnn_gguf_header_free(qnn_gguf_header *header) {
  delete header;
  return QNN_OK;
}

int qnn_gguf_header_get(const qnn_gguf_header *h, qnn_gguf_header_info *o) {
  if (!h || !o) return QNN_E_ARGUMENT;
  o->version = h->version;
  o->alignment = h->alignment;
  o->data_offset = h->data_offset;
  o->vocabulary_size = h->vocabulary_size;
  o->tensor_count = int32_t(h->tensors.size());
  o->architecture = h->architecture.c_str();
  o->metadata_json = h->metadata_json.c_str();
  return QNN_OK;
}

int qnn_gguf_header_tensor(const qnn_gguf_header *h, int index, qnn_gguf_tensor *o) {
  if (!h || !o || index < 0 || index >= int(h->tensors.size())) return QNN_E_ARGUMENT;
  const GgufTensor &t = h->tensors[index];
  o->name = t.name.c_str();
  o->shape = t.shape.data();
  o->offset = t.offset;
  o->byte_size = t.byte_size;
  o->ndim = int32_t(t.shape.size());
  o->storage_type = t.storage;
  o->encoding = t.encoding;
  return QNN_OK;
}

}  // extern "C"
