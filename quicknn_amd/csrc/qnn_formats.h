// qnn_formats.h -- checkpoint files on the host: safetensors and GGUF tensor
// tables (qnn_files.cpp) and the INT4 weight cache (qnn_int4_cache.cpp).
// Host-only C++: no HIP headers, built with the host compiler.
#pragma once

#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/qnn_hip.h"
#include "qnn_json.h"

namespace qnn {

// Sets the calling thread's qnn_last_error text (defined beside the context).
void set_last_error(const std::string &msg);

namespace fmt {

// An exception carrying a QNN_E_* code, converted to a status at the C ABI.
struct Error : std::runtime_error {
  int code;
  Error(int c, const std::string &m) : std::runtime_error(m), code(c) {}
};
[[noreturn]] inline void fail(int code, const std::string &msg) { throw Error(code, msg); }

template <typename F>
int guarded(F &&f) {
  try {
    return f();
  } catch (const Error &e) {
    set_last_error(e.what());
    return e.code;
  } catch (const std::bad_alloc &) {
    set_last_error("host allocation failed");
    return QNN_E_RANGE;
  } catch (const std::exception &e) {
    set_last_error(e.what());
    return QNN_E_INVALID_OP;
  }
}

// A read-only private mapping of a whole file, unmapped on destruction.
struct Mapping {
  void *addr = nullptr;
  size_t size = 0;
  ~Mapping();
};

// TSafeTensor (src/io/QuickNN.SafeTensors.pas:149-180).
struct Tensor {
  std::string name;
  std::vector<int64_t> shape;
  int32_t st_dtype = QNN_ST_UNKNOWN;  // TSafeTensorType ordinal
  int32_t encoding = QNN_WE_NATIVE;   // TQNNWeightEncoding ordinal
  uint32_t storage_type = 0xFFFFFFFFu;  // GGML type (GGUF only)
  int64_t data_offset = 0, data_size = 0;  // absolute file offset, bytes
  const uint8_t *data = nullptr;
  uint64_t identity = 0;
  int64_t count() const {
    int64_t c = 1;
    for (int64_t d : shape) c *= d;
    return c;
  }
};

// TSafeTensorFile (src/io/QuickNN.SafeTensors.pas:184-205).
struct File {
  std::string path, architecture;
  bool is_gguf = false;
  int64_t file_size = 0, header_size = 0, data_size = 0, offset = 0;
  std::string header_json;  // the raw header bytes (safetensors only)
  json::Value json;         // the parsed header (safetensors only)
  std::vector<Tensor> tensors;  // descriptor order
  std::vector<int> by_name;     // indices sorted by name
  std::shared_ptr<Mapping> map;
  // F32 copies made by GetLinearWeight for F16 tensors, kept while open.
  std::vector<std::pair<int, std::unique_ptr<float[]>>> converted;
  const Tensor *find(const std::string &name) const;
};

// TSafeTensorFiles: the files of one checkpoint, searched in order.
struct FileSet {
  std::vector<std::unique_ptr<File>> files;
  const Tensor *find(const std::string &name, int *file_index = nullptr) const;
};

std::unique_ptr<File> open_file(const std::string &path);
std::unique_ptr<FileSet> open_shards(const std::string &dir, const std::string &index_file,
                                     const std::string &single_file);
// Reads a whole text file, dropping a UTF-8 byte order mark.
std::string read_text(const std::string &path);
bool file_exists(const std::string &path);
std::string join_path(const std::string &dir, const std::string &name);
// Absolute, lexically normalised path ("." and ".." resolved, no symlinks followed).
std::string full_path(const std::string &path);
// A fresh non-zero WeightIdentity (top bit set, apart from caller-made ones).
uint64_t new_identity();

}  // namespace fmt
}  // namespace qnn

struct qnn_tensor_files_s : qnn::fmt::FileSet {};
