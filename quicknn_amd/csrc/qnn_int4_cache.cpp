// qnn_int4_cache.cpp -- the INT4 weight cache of an LLM checkpoint.
//
// Restates TLLMInt4Cache (src/models/QuickNN.Models.LLM.Quantization.pas):
//  * formats and index names (:40-44); a cache lives in
//    <directory>/<format>-<SHA-256 fingerprint of the sources> (:79-95);
//  * the fingerprint (:54-68) hashes the format, then per source file its
//    full path, byte size, UTC write time as yyyymmddhhnnsszzz and raw header;
//  * weight selection (:180-199): routed-expert gate/up/down matrices, or
//    (dense scope) every 2-D language-model and lm_head weight except the
//    linear-attention in_proj_a / in_proj_b;
//  * shard writing (:200-292): QuantizeInt4 of each matrix into safetensors
//    shards of 384 (experts) or 32 (dense) U8 [rows, Int4RowBytes(cols)]
//    tensors, header metadata {format, source_fingerprint}, padded with spaces
//    to 8 bytes, written as *.part and renamed; the index is written last, so
//    only a finished build is ever visible;
//  * index and shard validation on open (:114-162).
// Quantisation is qnn_quantize_int4 (the packer of QuantizeInt4,
// src/core/QuickNN.Quantization.Int4.pas:96-144), threaded over rows.
#include <fcntl.h>
#include <sys/file.h>
#include <sys/stat.h>
#include <sys/types.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstdio>
#include <cstring>
#include <ctime>
#include <random>

#include "qnn_formats.h"

namespace qnn {
namespace fmt {
namespace {

// ---------------------------------------------------------------- SHA-256
// FIPS 180-4, section 6.2.
class Sha256 {
 public:
  Sha256() {
    static const uint32_t h0[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a,
                                   0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
    std::memcpy(h_, h0, sizeof h_);
  }
  void update(const void *data, size_t n) {
    const uint8_t *p = static_cast<const uint8_t *>(data);
    total_ += n;
    while (n) {
      const size_t take = std::min(n, size_t(64) - fill_);
      std::memcpy(buf_ + fill_, p, take);
      fill_ += take;
      p += take;
      n -= take;
      if (fill_ == 64) {
        block(buf_);
        fill_ = 0;
      }
    }
  }
  void update(const std::string &s) { update(s.data(), s.size()); }
  std::string hex() {
    const uint64_t bits = total_ * 8;
    const uint8_t one = 0x80, zero = 0;
    update(&one, 1);
    while (fill_ != 56) update(&zero, 1);
    uint8_t len[8];
    for (int i = 0; i < 8; ++i) len[i] = uint8_t(bits >> (56 - 8 * i));
    update(len, 8);
    static const char *digits = "0123456789abcdef";
    std::string out;
    for (uint32_t w : h_)
      for (int i = 28; i >= 0; i -= 4) out += digits[(w >> i) & 15];
    return out;
  }

 private:
  uint32_t h_[8];
  uint8_t buf_[64];
  size_t fill_ = 0;
  uint64_t total_ = 0;

  static uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }
  void block(const uint8_t *b) {
    static const uint32_t k[64] = {
        0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
        0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
        0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
        0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
        0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
        0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
        0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
        0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2};
    uint32_t w[64];
    for (int i = 0; i < 16; ++i)
      w[i] = uint32_t(b[4 * i]) << 24 | uint32_t(b[4 * i + 1]) << 16 | uint32_t(b[4 * i + 2]) << 8 | b[4 * i + 3];
    for (int i = 16; i < 64; ++i) {
      const uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
      const uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
      w[i] = w[i - 16] + s0 + w[i - 7] + s1;
    }
    uint32_t a = h_[0], bb = h_[1], c = h_[2], d = h_[3], e = h_[4], f = h_[5], g = h_[6], h = h_[7];
    for (int i = 0; i < 64; ++i) {
      const uint32_t t1 = h + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) + k[i] + w[i];
      const uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & bb) ^ (a & c) ^ (bb & c));
      h = g;
      g = f;
      f = e;
      e = d + t1;
      d = c;
      c = bb;
      bb = a;
      a = t1 + t2;
    }
    h_[0] += a; h_[1] += bb; h_[2] += c; h_[3] += d;
    h_[4] += e; h_[5] += f; h_[6] += g; h_[7] += h;
  }
};

// ---------------------------------------------------------------- formats
const char *const kCacheFormat = "quicknn-moe-int4-g32-ls-v1";
const char *const kDenseFormat = "quicknn-dense-int4-g32-ls-v1";
const char *const kLegacyFormat = "envision-moe-int4-g32-ls-v1";
const char *const kExpertIndex = "experts.safetensors.index.json";
const char *const kDenseIndex = "weights.safetensors.index.json";
constexpr int kExpertsPerShard = 384;
constexpr int kDensePerShard = 32;

bool ends_with(const std::string &s, const char *suffix) {
  const size_t n = std::strlen(suffix);
  return s.size() >= n && s.compare(s.size() - n, n, suffix) == 0;
}
bool starts_with(const std::string &s, const char *prefix) { return s.rfind(prefix, 0) == 0; }

// IsExpert (LLM.Quantization.pas:46-53).
bool is_expert(const std::string &name) {
  return name.find(".mlp.experts.") != std::string::npos &&
         (ends_with(name, ".gate_proj.weight") || ends_with(name, ".up_proj.weight") ||
          ends_with(name, ".down_proj.weight"));
}

// The selection rule of Build (LLM.Quantization.pas:180-187).
bool selected(const Tensor &t, int scope) {
  if (scope == QNN_IQ_EXPERTS) return is_expert(t.name);
  return t.shape.size() == 2 && (t.name == "lm_head.weight" || starts_with(t.name, "model.language_model.")) &&
         ends_with(t.name, ".weight") && !ends_with(t.name, ".in_proj_a.weight") &&
         !ends_with(t.name, ".in_proj_b.weight");
}

// FormatDateTime('yyyymmddhhnnsszzz', TFile.GetLastWriteTimeUtc(path)).
std::string write_time_utc(const std::string &path) {
  struct stat st;
  if (stat(path.c_str(), &st) != 0) fail(QNN_E_IO, "Cannot read the write time of " + path);
  const time_t sec = st.st_mtim.tv_sec;
  struct tm tm;
  gmtime_r(&sec, &tm);
  char b[96];
  std::snprintf(b, sizeof b, "%04d%02d%02d%02d%02d%02d%03d", tm.tm_year + 1900, tm.tm_mon + 1, tm.tm_mday,
                tm.tm_hour, tm.tm_min, tm.tm_sec, int(st.st_mtim.tv_nsec / 1000000));
  return b;
}

// FingerprintForFormat (LLM.Quantization.pas:55-68).
std::string fingerprint(const FileSet &sources, const std::string &format) {
  Sha256 h;
  h.update(format);
  for (const auto &f : sources.files) {
    h.update(full_path(f->path));
    h.update(std::to_string(f->file_size));
    h.update(write_time_utc(f->path));
    h.update(f->header_json);
  }
  return h.hex();
}

std::string base_name(const std::string &p) {
  const size_t s = p.find_last_of('/');
  return s == std::string::npos ? p : p.substr(s + 1);
}
std::string dir_name(const std::string &p) {
  const size_t s = p.find_last_of('/');
  if (s == std::string::npos) return "";
  return s == 0 ? "/" : p.substr(0, s);
}
std::string lower(std::string s) {
  for (char &c : s)
    if (c >= 'A' && c <= 'Z') c = char(c - 'A' + 'a');
  return s;
}

void make_dirs(const std::string &path) {
  std::string cur;
  size_t pos = 0;
  while (pos != std::string::npos) {
    pos = path.find('/', pos + 1);
    cur = path.substr(0, pos);
    if (cur.empty()) continue;
    if (mkdir(cur.c_str(), 0777) != 0 && errno != EEXIST)
      fail(QNN_E_IO, "Cannot create directory " + cur + ": " + std::strerror(errno));
  }
}

std::string guid_name() {
  std::random_device rd;
  char b[64];
  std::snprintf(b, sizeof b, "{%08X-%04X-%04X-%04X-%04X%08X}", rd(), rd() & 0xffff, rd() & 0xffff, rd() & 0xffff,
                rd() & 0xffff, rd());
  return b;
}

void write_all(int fd, const void *data, size_t n, const std::string &path) {
  const uint8_t *p = static_cast<const uint8_t *>(data);
  while (n) {
    const ssize_t w = ::write(fd, p, n);
    if (w < 0) {
      if (errno == EINTR) continue;
      fail(QNN_E_IO, "Cannot write " + path + ": " + std::strerror(errno));
    }
    p += w;
    n -= size_t(w);
  }
}

// A file removed on scope exit unless released (a failed build publishes nothing).
struct TempFile {
  std::string path;
  int fd = -1;
  ~TempFile() {
    if (fd >= 0) close(fd);
    if (!path.empty()) unlink(path.c_str());
  }
  void commit(const std::string &target) {
    if (fd >= 0 && close(fd) != 0) {
      fd = -1;
      fail(QNN_E_IO, "Cannot close " + path);
    }
    fd = -1;
    if (rename(path.c_str(), target.c_str()) != 0)
      fail(QNN_E_IO, "Cannot rename " + path + " to " + target + ": " + std::strerror(errno));
    path.clear();
  }
};

}  // namespace

struct Int4Cache {
  std::unique_ptr<FileSet> files;
  std::string directory, fingerprint, format, index_name;
  int scope = QNN_IQ_EXPERTS;

  // Build (LLM.Quantization.pas:164-297).
  void build(const FileSet &sources, qnn_progress_fn progress, void *user) {
    std::vector<const Tensor *> tensors;
    for (const auto &f : sources.files)
      for (const Tensor &t : f->tensors)
        if (selected(t, scope)) {
          if (t.shape.size() != 2 || (t.st_dtype != QNN_ST_F32 && t.st_dtype != QNN_ST_BF16) || t.shape[0] < 1 ||
              t.shape[0] > 0x7fffffff || t.shape[1] < 1 || t.shape[1] > 0x7fffffff)
            fail(QNN_E_ARGUMENT, "Invalid native INT4 source: " + t.name);
          tensors.push_back(&t);
        }
    if (tensors.empty()) fail(QNN_E_ARGUMENT, "No native weights selected for INT4 conversion");
    const std::string meta = "{\"format\":" + json::quote(format) +
                             ",\"source_fingerprint\":" + json::quote(fingerprint) + "}";
    std::string map = "{";
    const int per_shard = scope == QNN_IQ_DENSE ? kDensePerShard : kExpertsPerShard;
    const int count = int(tensors.size());
    const int shards = (count + per_shard - 1) / per_shard;
    if (progress) progress(0, shards, user);
    for (int shard = 0; shard < shards; ++shard) {
      const int start = shard * per_shard, n = std::min(per_shard, count - start);
      char name[96];
      std::snprintf(name, sizeof name, "%s-%05d-of-%05d.safetensors", scope == QNN_IQ_DENSE ? "weights" : "experts",
                    shard + 1, shards);
      std::string header = "{\"__metadata__\":" + meta;
      int64_t offset = 0;
      for (int i = start; i < start + n; ++i) {
        const Tensor &t = *tensors[i];
        const int rb = qnn_int4_row_bytes(int(t.shape[1]));
        const int64_t bytes = t.shape[0] * rb;
        header += "," + json::quote(t.name) + ":{\"dtype\":\"U8\",\"shape\":[" + std::to_string(t.shape[0]) + "," +
                  std::to_string(rb) + "],\"data_offsets\":[" + std::to_string(offset) + "," +
                  std::to_string(offset + bytes) + "]}";
        offset += bytes;
        if (map.size() > 1) map += ",";
        map += json::quote(t.name) + ":" + json::quote(name);
      }
      header += "}";
      while (header.size() % 8 != 0) header += ' ';
      TempFile tmp;
      tmp.path = join_path(directory, guid_name() + ".part");
      tmp.fd = open(tmp.path.c_str(), O_WRONLY | O_CREAT | O_TRUNC | O_CLOEXEC, 0666);
      if (tmp.fd < 0) {
        tmp.path.clear();
        fail(QNN_E_IO, "Cannot create a shard in " + directory + ": " + std::strerror(errno));
      }
      const uint64_t header_bytes = header.size();
      write_all(tmp.fd, &header_bytes, 8, tmp.path);
      write_all(tmp.fd, header.data(), header.size(), tmp.path);
      std::vector<uint8_t> encoded;
      for (int i = start; i < start + n; ++i) {
        const Tensor &t = *tensors[i];
        const int rows = int(t.shape[0]), cols = int(t.shape[1]);
        encoded.resize(size_t(rows) * size_t(qnn_int4_row_bytes(cols)));
        const int rc = qnn_quantize_int4(t.data, t.st_dtype == QNN_ST_BF16 ? QNN_DT_BF16 : QNN_DT_F32, rows, cols,
                                         encoded.data());
        if (rc != QNN_OK) fail(rc, "QuantizeInt4 rejected " + t.name + " (non-finite values)");
        write_all(tmp.fd, encoded.data(), encoded.size(), tmp.path);
      }
      tmp.commit(join_path(directory, name));
      if (progress) progress(shard + 1, shards, user);
    }
    map += "}";
    if (fmt::fingerprint(sources, format) != fingerprint)
      fail(QNN_E_INVALID_OP, "Source weights changed during INT4 conversion");
    const std::string index = "\xEF\xBB\xBF{\"metadata\":" + meta + ",\"weight_map\":" + map + "}";
    TempFile tmp;
    tmp.path = join_path(directory, index_name + ".part");
    tmp.fd = open(tmp.path.c_str(), O_WRONLY | O_CREAT | O_TRUNC | O_CLOEXEC, 0666);
    if (tmp.fd < 0) {
      tmp.path.clear();
      fail(QNN_E_IO, "Cannot write the INT4 cache index in " + directory);
    }
    write_all(tmp.fd, index.data(), index.size(), tmp.path);
    tmp.commit(join_path(directory, index_name));
  }

  // ValidateIndex (LLM.Quantization.pas:137-162).
  void validate_index() const {
    const std::string text = read_text(join_path(directory, index_name));
    json::Value index;
    json::Parser parser(text.data(), text.size());
    if (!parser.parse(index) || !index.is_object() || index.string_at("metadata.format") != format ||
        index.string_at("metadata.source_fingerprint") != fingerprint)
      fail(QNN_E_FORMAT, "Invalid or stale INT4 cache index");
    const json::Value *map = index.get("weight_map");
    if (!map || !map->is_object()) fail(QNN_E_FORMAT, "Missing INT4 weight map");
    for (const auto &m : map->members) {
      const std::string &v = m.second.text;
      if (!m.second.is_string() || v.empty() || v.find_first_of(":/\\") != std::string::npos)
        fail(QNN_E_FORMAT, "Invalid INT4 shard path");
    }
  }
};

// TLLMInt4Cache.Create (LLM.Quantization.pas:79-125).
std::unique_ptr<Int4Cache> open_cache(const FileSet &sources, const std::string &directory, qnn_progress_fn progress,
                                      void *user, int scope) {
  if (directory.empty()) fail(QNN_E_ARGUMENT, "Missing INT4 cache directory");
  if (scope != QNN_IQ_EXPERTS && scope != QNN_IQ_DENSE) fail(QNN_E_ARGUMENT, "INT4 cache scope");
  auto c = std::make_unique<Int4Cache>();
  c->scope = scope;
  c->index_name = scope == QNN_IQ_DENSE ? kDenseIndex : kExpertIndex;
  c->format = scope == QNN_IQ_DENSE ? kDenseFormat : kCacheFormat;
  c->fingerprint = fingerprint(sources, c->format);
  const std::string root = full_path(directory);
  c->directory = join_path(root, c->format + "-" + c->fingerprint);
  if (scope == QNN_IQ_EXPERTS && !file_exists(join_path(c->directory, c->index_name))) {
    // A verified cache of the older format name is reused as it stands.
    std::string legacy_root = root;
    if (lower(base_name(legacy_root)) == ".quicknn-cache") legacy_root = join_path(dir_name(legacy_root), ".envision-cache");
    const std::string legacy_fp = fingerprint(sources, kLegacyFormat);
    const std::string legacy_dir = join_path(legacy_root, std::string(kLegacyFormat) + "-" + legacy_fp);
    if (file_exists(join_path(legacy_dir, c->index_name))) {
      c->directory = legacy_dir;
      c->fingerprint = legacy_fp;
      c->format = kLegacyFormat;
    }
  }
  if (!file_exists(join_path(c->directory, c->index_name))) {
    make_dirs(c->directory);
    // Only a committed index makes a cache visible; the exclusive lock keeps
    // two builders from publishing the same shard names.
    const std::string lock_path = join_path(c->directory, "build.lock");
    const int lock = open(lock_path.c_str(), O_RDWR | O_CREAT | O_TRUNC | O_CLOEXEC, 0666);
    if (lock < 0) fail(QNN_E_IO, "Cannot create " + lock_path + ": " + std::strerror(errno));
    if (flock(lock, LOCK_EX | LOCK_NB) != 0) {
      close(lock);
      fail(QNN_E_IO, "Cannot create " + lock_path + ": the INT4 cache is being built by another process");
    }
    try {
      if (!file_exists(join_path(c->directory, c->index_name))) c->build(sources, progress, user);
    } catch (...) {
      close(lock);
      throw;
    }
    close(lock);
  }
  c->validate_index();
  c->files = open_shards(c->directory, c->index_name, "");
  for (const auto &f : c->files->files)
    if (f->json.string_at("__metadata__.format") != c->format ||
        f->json.string_at("__metadata__.source_fingerprint") != c->fingerprint)
      fail(QNN_E_FORMAT, "Invalid INT4 shard format");
  return c;
}

}  // namespace fmt
}  // namespace qnn

struct qnn_int4_cache_s : qnn::fmt::Int4Cache {};

using namespace qnn::fmt;

extern "C" {

int qnn_int4_cache_create(const qnn_tensor_files *sources, const char *directory, qnn_progress_fn progress,
                          void *user, int scope, qnn_int4_cache **out) {
  return guarded([&] {
    if (!sources || !out) fail(QNN_E_ARGUMENT, "null argument");
    *out = nullptr;
    auto c = open_cache(*static_cast<const FileSet *>(sources), directory ? directory : "", progress, user,
                        scope);
    auto h = std::make_unique<qnn_int4_cache_s>();
    static_cast<Int4Cache &>(*h) = std::move(*c);
    *out = h.release();
    return QNN_OK;
  });
}

int qnn_int4_cache_destroy(qnn_int4_cache *cache) {
  delete cache;
  return QNN_OK;
}

int qnn_int4_cache_weight(const qnn_int4_cache *cache, const char *name, int rows, int columns, qnn_weight *o) {
  return guarded([&] {
    if (!cache || !name || !o) fail(QNN_E_ARGUMENT, "null argument");
    const int rb = qnn_int4_row_bytes(columns);
    if (rb < 0) fail(QNN_E_ARGUMENT, "INT4 matrix width");
    const Tensor *t = cache->files ? cache->files->find(name) : nullptr;
    if (!t || t->st_dtype != QNN_ST_U8 || t->shape.size() != 2 || t->shape[0] != rows || t->shape[1] != rb)
      fail(QNN_E_FORMAT, std::string("Missing or invalid packed INT4 weight: ") + name);
    std::memset(o, 0, sizeof *o);
    o->identity = t->identity;
    o->data = t->data;
    o->offset = 0;
    o->size = t->count();
    o->shape0 = t->shape[0];
    o->shape1 = t->shape[1];
    o->dtype = QNN_DT_U8;
    o->encoding = QNN_WE_NATIVE;
    return QNN_OK;
  });
}

int qnn_int4_cache_mapped_bytes(const qnn_int4_cache *cache, uint64_t *bytes) {
  if (!cache || !bytes) return QNN_E_ARGUMENT;
  uint64_t total = 0;
  if (cache->files)
    for (const auto &f : cache->files->files) total += uint64_t(f->data_size);
  *bytes = total;
  return QNN_OK;
}

const char *qnn_int4_cache_directory(const qnn_int4_cache *cache) {
  return cache ? cache->directory.c_str() : "";
}

int qnn_int4_source_fingerprint(const qnn_tensor_files *sources, char *out) {
  return guarded([&] {
    if (!sources || !out) fail(QNN_E_ARGUMENT, "null argument");
    const std::string fp = fingerprint(*static_cast<const FileSet *>(sources), kCacheFormat);
    std::memcpy(out, fp.c_str(), fp.size() + 1);
    return QNN_OK;
  });
}

}  // extern "C"
